"""Within-block variance of a flat tensor for one period, on the MI355X.

Same public names as the reference module kernels/period_variance.py:
``average_within_block_variance_cuda_kernel(values, period, *,
input_is_squared) -> float`` (reference :62-85) and the torch custom op
``gefen::average_within_block_variance_cuda`` (reference :36-57), which
returns a 0-dim fp32 device tensor and keeps the call in a traced graph.
Both are one C-ABI call, ``gefenx_block_variance_errors_ex``: the result is
sqrt(mean over blocks of var(x)), x = fp32(value)^2 (or fp32(value) when the
input already holds squares), accumulated in float64 with a two-pass variance
per block.  The reference kernel uses fp32 one-pass sums with float atomics,
so last bits can differ; the period search (partitioning.py) compares these
errors, and its device backend (gefenx_block_variance_errors) batches all
divisors of a tensor in one call.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _native

_OPAQUE_OP_AVAILABLE = False


def _errors(values: torch.Tensor, period: int, input_is_squared: bool) -> float:
    from .automatic_gefen_fused import _dtype_code, _stream
    flat = values.detach().reshape(-1)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    per = np.array([int(period)], dtype=np.int64)
    out = np.zeros(1, dtype=np.float64)
    _native.check(_native.load().gefenx_block_variance_errors_ex(
        flat.data_ptr(), _dtype_code(flat.dtype), flat.numel(), per.ctypes.data, 1,
        1 if input_is_squared else 0, out.ctypes.data, _stream(flat.device)),
        "average_within_block_variance_cuda")
    return float(out[0])


def _average_within_block_variance_cuda_impl(values: torch.Tensor, period: int,
                                             input_is_squared: bool) -> torch.Tensor:
    """0-dim fp32 tensor on the values' device (the reference op's result)."""
    err = _errors(values, period, input_is_squared)
    return torch.tensor(err, dtype=torch.float32, device=values.device)


if hasattr(torch.library, "custom_op"):

    @torch.library.custom_op("gefen::average_within_block_variance_cuda", mutates_args=())
    def _average_within_block_variance_cuda_opaque(values: torch.Tensor, period: int,
                                                   input_is_squared: bool) -> torch.Tensor:
        return _average_within_block_variance_cuda_impl(values, period, input_is_squared)

    @_average_within_block_variance_cuda_opaque.register_fake
    def _average_within_block_variance_cuda_opaque_fake(values: torch.Tensor, period: int,
                                                        input_is_squared: bool) -> torch.Tensor:
        del period, input_is_squared
        return values.new_empty((), dtype=torch.float32)

    _OPAQUE_OP_AVAILABLE = True


def average_within_block_variance_cuda_kernel(values: torch.Tensor, period: int, *,
                                              input_is_squared: bool) -> float:
    """Reference kernels/period_variance.py:62-85: same argument checks and
    exception types, then the device computation."""
    if not isinstance(values, torch.Tensor):
        raise TypeError("Expected torch.Tensor, got {}".format(type(values).__name__))
    elif values.device.type != "cuda":
        raise ValueError("Expected a CUDA tensor, got device {}".format(values.device))
    elif values.numel() == 0:
        raise ValueError("Expected a non-empty tensor.")
    elif period <= 0:
        raise ValueError("Expected a positive period, got {}".format(period))
    elif values.numel() % period != 0:
        raise ValueError("Expected length {} to be divisible by period {}.".format(values.numel(), period))
    if values.dtype == torch.float64:
        raise NotImplementedError("average_within_block_variance_cuda: fp32/fp16/bf16 inputs only")
    return _errors(values, int(period), bool(input_is_squared))
