"""Block-period search (reference partitioning.py).

Same public functions and rule as the reference: candidate periods are the
proper divisors of numel; each candidate's error is the square root of the mean
within-block variance of g^2; the chosen period is the one after the largest
error drop (partitioning.py:237-271), periods below 8 collapse to 1 and then to
the memory-safe fallback (partitioning.py:31-47).

Backends: "cpu" (numpy float64, the reference's CPU arithmetic) and
"cuda_kernel" (the MI355X C ABI: every candidate's error in float64 on the GPU,
one host sync for all candidates instead of one per divisor).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

MEMORY_SAFE_FALLBACK = True
FALLBACK_PERIOD_CAP = 2048


def _largest_divisor_at_most(n, cap):
    best = 1
    for i in range(1, int(n ** 0.5) + 1):
        if n % i == 0:
            if cap >= i > best:
                best = i
            j = n // i
            if cap >= j > best:
                best = j
    return best


def memory_safe_fallback_period(n, parameter_shape):
    if n < 8:
        return 1
    candidates = []
    if parameter_shape is not None and len(parameter_shape) >= 2:
        in_features = int(parameter_shape[-1])
        if in_features >= 8 and n % in_features == 0:
            candidates.append(in_features)
    capped = _largest_divisor_at_most(n, FALLBACK_PERIOD_CAP)
    if capped >= 8:
        candidates.append(capped)
    if not candidates:
        return 1
    return max(candidates)


def divisors(n):
    small, large = [], []
    for i in range(1, int(n ** 0.5) + 1):
        if n % i == 0:
            if i != n:
                small.append(i)
            if i != n // i and n // i != n:
                large.append(n // i)
    return small + large[::-1]


def average_within_block_variance_cpu(list_of_values, period_to_check, parameter_name=None,
                                      parameter_shape=None):
    values = np.asarray(list_of_values, dtype=float)
    n = len(values)
    if n % period_to_check != 0:
        raise ValueError("Expected length {} to be divisible by period {}.".format(n, period_to_check))
    return np.sqrt(values.reshape(-1, period_to_check).var(axis=1).mean())


def average_within_block_variance_torch(values, period, parameter_name=None, parameter_shape=None):
    """Reference partitioning.py:87-108: sqrt(mean over blocks of each
    block's population variance) of a tensor's values.  A tensor on a HIP
    device is reduced by the block-variance kernel (float64 sums), a host
    tensor by the float64 restatement above."""
    if not isinstance(values, torch.Tensor):
        raise TypeError("Expected torch.Tensor, got {}".format(type(values).__name__))
    flat = values.detach().reshape(-1)
    n = flat.numel()
    if n % period != 0:
        raise ValueError("Expected length {} to be divisible by period {}.".format(n, period))
    if flat.device.type == "cuda":
        return block_variance_errors_device(flat.to(torch.float32), [int(period)], input_is_squared=True)[0]
    return float(average_within_block_variance_cpu(flat.to(torch.float64).numpy(), period))


def _finalize_period_results(list_periods_and_errors, print_results):
    if len(list_periods_and_errors) == 0:
        raise ValueError("Expected at least one valid period candidate.")
    scored = []
    previous_err = None
    for p, err in list_periods_and_errors:
        weighted = 1e-12 if previous_err is None else err - previous_err
        previous_err = err
        scored.append((p, err, weighted))
    if print_results:
        best_w = min(w for _, _, w in scored)
        for p, err, w in scored:
            line = f"p={p} |  err={err:.15f} | weighted error = {w:.15f}"
            print(f"\033[92m{line}\033[0m" if w == best_w else line)
    _, best_period = min((w, p) for p, _, w in scored)
    if best_period < 8:
        best_period = 1
    return best_period


def _find_period_cpu(squared_values, print_results=True):
    values = np.asarray(squared_values, dtype=float)
    results = [(p, average_within_block_variance_cpu(values, p)) for p in divisors(len(values))]
    if not results:
        raise ValueError("Could not find any valid period candidates.")
    return _finalize_period_results(results, print_results)


def block_variance_errors_device(grad: torch.Tensor, periods, input_is_squared: bool = False):
    """Errors of every candidate period for a device tensor (C ABI, one
    sync); the values are squared first unless input_is_squared."""
    from gefen.kernels import _native
    from gefen.kernels.automatic_gefen_fused import _dtype_code, _stream
    flat = grad.detach().reshape(-1)
    if not flat.is_contiguous():
        flat = flat.contiguous()
    per = np.ascontiguousarray(np.asarray(periods, dtype=np.int64))
    out = np.zeros(max(1, per.size), dtype=np.float64)
    _native.check(_native.load().gefenx_block_variance_errors_ex(
        flat.data_ptr(), _dtype_code(flat.dtype), flat.numel(), per.ctypes.data, int(per.size),
        1 if input_is_squared else 0, out.ctypes.data, _stream(flat.device)), "block variance errors")
    return [float(e) for e in out[: per.size]]


def _find_period_device(grad: torch.Tensor, print_results=True, input_is_squared=False):
    if not isinstance(grad, torch.Tensor):
        raise TypeError("Expected torch.Tensor for the device backends, got {}".format(type(grad).__name__))
    if grad.device.type != "cuda":
        raise ValueError("Expected a CUDA tensor for the device backends, got device {}".format(grad.device))
    divs = divisors(grad.numel())
    if not divs:
        raise ValueError("Could not find any valid period candidates.")
    errs = block_variance_errors_device(grad, divs, input_is_squared)
    return _finalize_period_results(list(zip(divs, errs)), print_results)


def find_period_by_block_variance(squared_grad_flattened_values, print_results=True,
                                  parameter_name=None, parameter_shape=None, backend="cpu",
                                  input_is_squared=True):
    """Reference partitioning.py:274-313.  "gpu" (the reference's torch
    backend, always on squared values) and "cuda_kernel" (squared values,
    or with input_is_squared=False the raw grad, squared by the kernel) both
    run the block-variance kernel over all candidate periods at once."""
    if backend == "cpu":
        period = _find_period_cpu(squared_grad_flattened_values, print_results)
        n = len(np.asarray(squared_grad_flattened_values).reshape(-1))
    elif backend in ("cuda_kernel", "gpu"):
        squared = True if backend == "gpu" else bool(input_is_squared)
        period = _find_period_device(squared_grad_flattened_values, print_results, input_is_squared=squared)
        n = int(squared_grad_flattened_values.numel())
    else:
        raise ValueError("Unexpected backend: {}".format(backend))
    if MEMORY_SAFE_FALLBACK and period == 1:
        return memory_safe_fallback_period(n, parameter_shape)
    return period
