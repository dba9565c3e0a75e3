"""Block vmean EMA on the GPU: the Python surface of the reference module
kernels/automatic_vmean.py (`automatic_vmean_update_cuda`, `_load_extension`),
backed by gefenx_vmean_update of the C ABI (include/gefenx.h).

vmean[b] <- fma(mean_b, 1-beta2, vmean[b]*beta2), mean_b the mean of the
block's squared grads; bf16 grads square and average through bf16 as the
reference's decomposed step does (gefen.py:129-191), which is the arithmetic
the oracle pins.
"""
from __future__ import annotations

import torch

from . import _native
from .automatic_gefen_fused import _dtype_code, _stream


class _Extension:
    """Reference binding surface (kernels/automatic_vmean_binding.cpp)."""

    @staticmethod
    def automatic_vmean_update_cuda(vmean: torch.Tensor, grad_view: torch.Tensor, beta2: float) -> None:
        if vmean.device.type != "cuda" or grad_view.device.type != "cuda":
            raise ValueError("Expected vmean and grad_view to be on CUDA.")
        if not vmean.is_contiguous():
            raise ValueError("Expected vmean to be contiguous.")
        if not grad_view.is_contiguous():
            raise ValueError("Expected grad_view to be contiguous.")
        if grad_view.dim() != 2:
            raise ValueError("Expected grad_view to be 2D.")
        if vmean.dim() != 2 or vmean.size(1) != 1:
            raise ValueError("Expected vmean to have shape [num_blocks, 1].")
        if vmean.dtype != torch.float32:
            raise ValueError("Expected vmean to have dtype float32.")
        num_blocks, period = grad_view.shape
        if vmean.size(0) != num_blocks:
            raise ValueError("Expected vmean and grad_view to have the same number of blocks.")
        if period <= 0:
            raise ValueError("Expected grad_view to have a positive period.")
        if num_blocks == 0:
            return
        _native.check(_native.load().gefenx_vmean_update(
            vmean.data_ptr(), grad_view.data_ptr(), _dtype_code(grad_view.dtype), grad_view.numel(), period,
            float(beta2), _stream(vmean.device)), "automatic_vmean_update_cuda")


_EXTENSION_MODULE = None


def _load_extension() -> _Extension:
    """Reference kernels/automatic_vmean.py:8-20."""
    global _EXTENSION_MODULE
    if _EXTENSION_MODULE is None:
        _native.load()
        _EXTENSION_MODULE = _Extension()
    return _EXTENSION_MODULE


def automatic_vmean_update_cuda(vmean: torch.Tensor, grad_view: torch.Tensor, beta2: float) -> None:
    """Reference kernels/automatic_vmean.py:23-41: reject a device mismatch,
    make the grad contiguous, update vmean in place."""
    if grad_view.device != vmean.device:
        raise ValueError("grad_view device {} must match vmean device {}.".format(grad_view.device, vmean.device))
    grad_c = grad_view if grad_view.is_contiguous() else grad_view.contiguous()
    _load_extension().automatic_vmean_update_cuda(vmean, grad_c, beta2)
