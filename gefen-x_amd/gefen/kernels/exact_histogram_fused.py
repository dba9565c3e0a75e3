"""Step-1 histogram on the GPU: the Python surface of the reference module
kernels/exact_histogram_fused.py (`gefen_exact_histogram_cuda`,
`_load_extension`), backed by gefenx_exact_histogram of the C ABI.

Every grad is divided by the absolute maximum of its block (a block whose
maximum is 0 contributes zeros), binned as clamp(floor((x + 1) / (2 / bins)),
0, bins - 1), and the counts are added into `bin_counts` (int64, accumulated
across calls) -- the bincount of gefen.py:455-469.
"""
from __future__ import annotations

import torch

from . import _native
from .automatic_gefen_fused import _dtype_code, _stream


class _Extension:
    """Reference binding surface (kernels/exact_histogram_fused_binding.cpp)."""

    @staticmethod
    def gefen_exact_histogram_cuda(grad_flat: torch.Tensor, period: int, bin_counts: torch.Tensor) -> None:
        if not grad_flat.is_contiguous():
            raise ValueError("Expected grad_flat to be contiguous.")
        if grad_flat.numel() == 0:
            return
        _native.check(_native.load().gefenx_exact_histogram(
            grad_flat.data_ptr(), _dtype_code(grad_flat.dtype), grad_flat.numel(), int(period),
            bin_counts.data_ptr(), bin_counts.numel(), _stream(grad_flat.device)), "gefen_exact_histogram_cuda")


_EXTENSION_MODULE = None


def _load_extension() -> _Extension:
    """Reference kernels/exact_histogram_fused.py:8-20."""
    global _EXTENSION_MODULE
    if _EXTENSION_MODULE is None:
        _native.load()
        _EXTENSION_MODULE = _Extension()
    return _EXTENSION_MODULE


def gefen_exact_histogram_cuda(grad_flat: torch.Tensor, period: int, bin_counts: torch.Tensor) -> None:
    """Reference kernels/exact_histogram_fused.py:23-79: the same argument
    checks (types, devices, ranks, dtype, period, divisibility, 1..4096
    bins) with the same exception types, then the histogram."""
    for name, tensor in (("grad_flat", grad_flat), ("bin_counts", bin_counts)):
        if not isinstance(tensor, torch.Tensor):
            raise TypeError("Expected {} to be a torch.Tensor.".format(name))
        if tensor.device.type != "cuda":
            raise ValueError("Expected {} to be on CUDA, got device {}.".format(name, tensor.device))
    if grad_flat.device != bin_counts.device:
        raise ValueError("Expected grad_flat and bin_counts on the same device, got {} and {}.".format(
            grad_flat.device, bin_counts.device))
    if grad_flat.dim() != 1:
        raise ValueError("Expected grad_flat to be 1D, got dim={}".format(grad_flat.dim()))
    if bin_counts.dim() != 1:
        raise ValueError("Expected bin_counts to be 1D, got dim={}".format(bin_counts.dim()))
    if bin_counts.dtype != torch.int64:
        raise ValueError("Expected bin_counts to be int64, got {}".format(bin_counts.dtype))
    if period <= 0:
        raise ValueError("Expected period to be positive, got {}".format(period))
    if grad_flat.numel() % period != 0:
        raise ValueError("Expected grad_flat.numel()={} to be divisible by period={}.".format(
            grad_flat.numel(), period))
    if bin_counts.numel() <= 0 or bin_counts.numel() > 4096:
        raise ValueError("Expected histogram bins in [1, 4096], got {}".format(bin_counts.numel()))
    _load_extension().gefen_exact_histogram_cuda(grad_flat.contiguous(), period, bin_counts)
