"""Python surface of the fused Gefen kernels, backed by the MI355X C ABI.

Same public names and signatures as the reference module
kernels/automatic_gefen_fused.py (automatic_gefen_fused_full_update_cuda,
automatic_gefen_fused_update_v2_full_cuda, gefen_factored_update_cuda,
gefen_quantized_momentum_update_cuda, _codebook_search_lut, _should_use_v2,
_should_use_v2_full, _CAPT_V1_FULL_TINY_NUMEL, ensure_extension_loaded), so
the optimizer and the reference's tests call them unchanged.  Underneath, every
call is one C-ABI function (include/gefenx.h) enqueued on torch's current HIP
stream; nothing here computes on the host.
"""
from __future__ import annotations

import ctypes
import os
import warnings
from typing import Optional

import torch

from . import _native

_LUT_BUCKETS = 4096
_LUT_CACHE: dict = {}

# Routing constants of the reference (kernels/automatic_gefen_fused.py:23-50).
# This build has ONE block-path kernel set; the predicates are kept because
# the optimizer and tests consult them, and both routes reach the same kernels.
_V2_PERIOD_MAX = 16
_V2_BLOCKS_PER_SM = 2
_CAPT_V1_FULL_TINY_NUMEL = 1 << 14
_FULL_V1_PERIOD_MIN = 16
_FULL_V1_PERIOD_MAX = 2048
_FULL_V1_TINY_NUM_BLOCKS = 1 << 13
_FULL_V2_LARGE_PERIOD_MIN = 1 << 13
_FULL_V2_PERIOD16_NUMEL = 1 << 24
_SM_COUNT_BY_DEVICE: dict = {}

_DTYPE_CODE = {torch.float32: _native.DT_F32, torch.float16: _native.DT_F16,
               torch.bfloat16: _native.DT_BF16, torch.float64: _native.DT_F64}


def _env_override(name: str) -> Optional[str]:
    value = os.environ.get(name)
    if value is None:
        return None
    value = value.strip()
    return value if value else None


_GEFEN_UPDATE_V2_ENV = _env_override("GEFEN_UPDATE_V2")


def ensure_extension_loaded() -> None:
    """Load the gfx950 library now, raising on failure (reference :139-148)."""
    _native.load()


def _dtype_code(dtype: torch.dtype) -> int:
    code = _DTYPE_CODE.get(dtype)
    if code is None:
        raise ValueError("unsupported dtype {}".format(dtype))
    return code


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _host_codebook(codebook: torch.Tensor):
    cb = codebook.detach().reshape(-1).to(device="cpu", dtype=torch.float32).contiguous()
    return cb


def _codebook_search_lut(codebook: torch.Tensor) -> torch.Tensor:
    """int16 [4097] search LUT on the codebook's device: lut[b] = #entries whose
    bucket < b (reference kernels/automatic_gefen_fused.py:81-121).  Built by
    the C ABI on the host once per (codebook storage, version, device)."""
    key = (codebook.data_ptr(), codebook._version, codebook.device)
    cached = _LUT_CACHE.get(key)
    if cached is not None:
        return cached[1]
    cb = _host_codebook(codebook)
    lut = torch.empty(_LUT_BUCKETS + 1, dtype=torch.int16)
    _native.check(_native.load().gefenx_search_lut(cb.data_ptr(), cb.numel(), _LUT_BUCKETS,
                                                   lut.data_ptr()), "search lut")
    lut = lut.to(codebook.device)
    while len(_LUT_CACHE) >= 16:
        _LUT_CACHE.pop(next(iter(_LUT_CACHE)))
    _LUT_CACHE[key] = (codebook, lut)
    return lut


def quant_table(codebook: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """Device byte image of the quantisation table for (codebook, grad dtype).
    One host build + one upload per codebook version (the exact-DP codebook is
    frozen after step 1).  The table is kept on the codebook tensor itself, so
    it lives exactly as long as the codebook: a captured graph that baked its
    address keeps working while the optimizer holds that codebook."""
    key = (codebook._version, codebook.device, dtype)
    cache = getattr(codebook, "_gefenx_qtables", None)
    if cache is not None and key in cache:
        return cache[key]
    lib = _native.load()
    cb = _host_codebook(codebook)
    if cb.numel() < 1 or cb.numel() > 256:
        raise ValueError("codebook must hold 1..256 entries, got {}".format(cb.numel()))
    host = torch.empty(int(lib.gefenx_qtable_bytes()), dtype=torch.uint8)
    _native.check(lib.gefenx_qtable_build(cb.data_ptr(), cb.numel(), _dtype_code(dtype),
                                          host.data_ptr()), "qtable build")
    dev = host.to(codebook.device) if codebook.device.type != "cpu" else host
    if cache is None:
        cache = {}
        codebook._gefenx_qtables = cache
    cache[key] = dev
    return dev


def workspace_for(anchor: torch.Tensor, kind: int, rows: int, cols: int, num_blocks: int) -> torch.Tensor:
    """Zero-initialised device workspace cached on the state tensor `anchor`
    (it lives exactly as long as the state); the kernels leave every
    accumulator zeroed after each call, so it is reused across steps."""
    nbytes = int(_native.load().gefenx_workspace_bytes(kind, rows, cols, num_blocks))
    cache = getattr(anchor, "_gefenx_ws", None)
    ws = None if cache is None else cache.get(kind)
    if ws is None or ws.numel() < nbytes or ws.device != anchor.device:
        ws = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=anchor.device)
        if cache is None:
            cache = {}
            anchor._gefenx_ws = cache
        cache[kind] = ws
    return ws


def _sm_count(device: torch.device) -> int:
    index = device.index if device.index is not None else torch.cuda.current_device()
    cached = _SM_COUNT_BY_DEVICE.get(index)
    if cached is None:
        cached = torch.cuda.get_device_properties(index).multi_processor_count
        _SM_COUNT_BY_DEVICE[index] = cached
    return cached


def _should_use_v2(num_blocks: int, period: int, device: torch.device) -> bool:
    """Legacy occupancy predicate (reference :162-173); env GEFEN_UPDATE_V2 overrides."""
    if _GEFEN_UPDATE_V2_ENV is not None:
        return _GEFEN_UPDATE_V2_ENV.lower() not in {"0", "false", "no", "off"}
    if period <= _V2_PERIOD_MAX:
        return True
    if device.type != "cuda":
        return False
    return num_blocks < _V2_BLOCKS_PER_SM * _sm_count(device)


def _should_use_v2_full(num_blocks: int, period: int, device: torch.device) -> bool:
    """Full-update route predicate (reference :176-199).  Both answers reach the
    same MI355X kernels here; the value is kept for callers that log it."""
    if _GEFEN_UPDATE_V2_ENV is not None:
        return _GEFEN_UPDATE_V2_ENV.lower() not in {"0", "false", "no", "off"}
    numel = num_blocks * period
    if period <= 15 and num_blocks <= _FULL_V1_TINY_NUM_BLOCKS:
        return False
    if period >= _FULL_V2_LARGE_PERIOD_MIN:
        return True
    if _FULL_V1_PERIOD_MIN <= period <= _FULL_V1_PERIOD_MAX:
        if period == 16 and numel >= _FULL_V2_PERIOD16_NUMEL:
            return True
        return False
    return _should_use_v2(num_blocks, period, device)


def _check_common(p, grad_view, m_sign, m_magnitude, codebook, packed_indices=False):
    if packed_indices:
        raise ValueError("packed_indices must be false: the 8-bit codebook stores one index per byte")
    if grad_view.dtype != p.dtype:
        raise ValueError("grad_view dtype {} must match p dtype {}.".format(grad_view.dtype, p.dtype))
    for name, t in (("grad_view", grad_view), ("m_sign", m_sign),
                    ("m_magnitude", m_magnitude), ("codebook", codebook)):
        if t.device != p.device:
            raise ValueError("{} device {} must match p device {}.".format(name, t.device, p.device))
    if p.device.type != "cuda":
        raise ValueError("fused Gefen kernels require HIP device tensors, got {}".format(p.device))
    if m_magnitude.dtype != torch.float32 or codebook.dtype != torch.float32:
        raise ValueError("m_magnitude and codebook must be float32.")
    if m_sign.dtype != torch.uint8:
        raise ValueError("m_sign must be uint8, got {}".format(m_sign.dtype))
    if p.dtype == torch.float64:
        raise NotImplementedError("Gefen fused kernels are not implemented for 'Double'")
    if grad_view.numel() != p.numel() or m_sign.numel() != p.numel():
        raise ValueError("grad_view / m_sign numel must equal p numel ({}).".format(p.numel()))
    if not m_sign.is_contiguous() or not m_magnitude.is_contiguous():
        raise ValueError("m_sign and m_magnitude must be contiguous.")


def _period_of(grad_view: torch.Tensor, m_magnitude: torch.Tensor) -> int:
    if grad_view.dim() == 2:
        period = int(grad_view.shape[1])
    else:
        period = grad_view.numel() // max(1, m_magnitude.numel())
    if period <= 0 or grad_view.numel() % period != 0 or m_magnitude.numel() * period != grad_view.numel():
        raise ValueError("m_magnitude ({}) does not match grad_view blocks {}".format(
            m_magnitude.numel(), tuple(grad_view.shape)))
    return period


def _scalar_ptrs(step_scalars, seed_dev):
    if step_scalars is not None:
        if step_scalars.dtype != torch.float32 or step_scalars.numel() < 4 or not step_scalars.is_contiguous():
            raise ValueError("step_scalars must be a contiguous float32 tensor with >= 4 entries")
    if seed_dev is not None:
        if seed_dev.dtype != torch.int64 or seed_dev.numel() < 1:
            raise ValueError("seed_dev must be an int64 tensor with >= 1 entry")
    return _ptr(step_scalars), _ptr(seed_dev)


def _strides_2d(t: torch.Tensor, rows: int, cols: int):
    if t.dim() == 2:
        return int(t.stride(0)), int(t.stride(1))
    if t.is_contiguous():
        return cols, 1
    raise ValueError("expected a 2D tensor or a contiguous tensor")


def _factored_update_impl(p: torch.Tensor, grad_view: torch.Tensor, m_sign: torch.Tensor,
                          m_magnitude: torch.Tensor, v_row: torch.Tensor, v_col: torch.Tensor,
                          codebook: torch.Tensor, cols: int, beta1: float, beta2: float, lr: float,
                          eps: float, inv_bias_correction_2: float, inv_bias_correction_1: float,
                          weight_decay_factor: float, stochastic_round: bool = False, rng_seed: int = 0,
                          step_scalars: Optional[torch.Tensor] = None,
                          codebook_lut: Optional[torch.Tensor] = None,
                          seed_dev: Optional[torch.Tensor] = None) -> None:
    _check_common(p, grad_view, m_sign, m_magnitude, codebook)
    cols = int(cols)
    numel = p.numel()
    if numel == 0:
        return
    if cols <= 0 or numel % cols != 0:
        raise ValueError("cols {} does not divide numel {}".format(cols, numel))
    rows = numel // cols
    if v_row.numel() != rows or v_col.numel() != cols:
        raise ValueError("v_row/v_col sizes ({}, {}) do not match [{}, {}]".format(
            v_row.numel(), v_col.numel(), rows, cols))
    if v_row.dtype != torch.float32 or v_col.dtype != torch.float32:
        raise ValueError("v_row and v_col must be float32")
    period = _period_of(grad_view, m_magnitude)
    grad_c = grad_view if grad_view.is_contiguous() else grad_view.contiguous()
    ps0, ps1 = _strides_2d(p, rows, cols)
    ss, sd = _scalar_ptrs(step_scalars, seed_dev)
    qt = quant_table(codebook, p.dtype)
    ws = workspace_for(m_magnitude, _native.WS_FACTORED, rows, cols, m_magnitude.numel())
    lib = _native.load()
    _native.check(lib.gefenx_factored_update(
        p.data_ptr(), grad_c.data_ptr(), _dtype_code(p.dtype), rows, cols, ps0, ps1, cols, 1,
        m_sign.data_ptr(), m_magnitude.data_ptr(), v_row.data_ptr(), v_col.data_ptr(), period,
        qt.data_ptr(), float(beta1), float(beta2), float(lr), float(eps),
        float(inv_bias_correction_2), float(inv_bias_correction_1), float(weight_decay_factor),
        1 if stochastic_round else 0, int(rng_seed), ss, sd, ws.data_ptr(), ws.numel(),
        _stream(p.device)), "gefen_factored_update_cuda")


def _block_update(p, grad_view, m_sign, m_magnitude, vmean, codebook, packed_indices, beta1,
                  beta2, lr, eps, inv_sqrt_bc2, inv_bc1, wdf, stochastic_round, rng_seed,
                  step_scalars, seed_dev, what):
    _check_common(p, grad_view, m_sign, m_magnitude, codebook, packed_indices)
    if p.numel() == 0:
        return
    if vmean.dtype != torch.float32 or vmean.numel() != m_magnitude.numel():
        raise ValueError("vmean must be float32 with one entry per block")
    if not p.is_contiguous():
        raise ValueError("p must be contiguous on the block path")
    period = _period_of(grad_view, m_magnitude)
    grad_c = grad_view if grad_view.is_contiguous() else grad_view.contiguous()
    ss, sd = _scalar_ptrs(step_scalars, seed_dev)
    qt = quant_table(codebook, p.dtype)
    ws = workspace_for(m_magnitude, _native.WS_BLOCK, 1, p.numel(), m_magnitude.numel())
    lib = _native.load()
    _native.check(lib.gefenx_block_update(
        p.data_ptr(), grad_c.data_ptr(), _dtype_code(p.dtype), p.numel(), period,
        m_sign.data_ptr(), m_magnitude.data_ptr(), vmean.data_ptr(), qt.data_ptr(),
        float(beta1), float(beta2), float(lr), float(eps), float(inv_sqrt_bc2), float(inv_bc1),
        float(wdf), 1 if stochastic_round else 0, int(rng_seed), ss, sd, ws.data_ptr(),
        ws.numel(), _stream(p.device)), what)


def _fused_full_update_impl(p: torch.Tensor, grad_view: torch.Tensor, m_sign: torch.Tensor,
                            m_magnitude: torch.Tensor, vmean: torch.Tensor, codebook: torch.Tensor,
                            packed_indices: bool, beta1: float, beta2: float, lr: float, eps: float,
                            inv_sqrt_bias_correction_2: float, inv_bias_correction_1: float,
                            weight_decay_factor: float, stochastic_round: bool = False, rng_seed: int = 0,
                            step_scalars: Optional[torch.Tensor] = None,
                            codebook_lut: Optional[torch.Tensor] = None,
                            seed_dev: Optional[torch.Tensor] = None) -> None:
    _block_update(p, grad_view, m_sign, m_magnitude, vmean, codebook, packed_indices, beta1,
                  beta2, lr, eps, inv_sqrt_bias_correction_2, inv_bias_correction_1,
                  weight_decay_factor, stochastic_round, rng_seed, step_scalars, seed_dev,
                  "automatic_gefen_fused_full_update_cuda")


def _fused_update_v2_full_impl(p: torch.Tensor, grad_view: torch.Tensor, m_sign: torch.Tensor,
                               m_magnitude: torch.Tensor, vmean: torch.Tensor, codebook: torch.Tensor,
                               packed_indices: bool, beta1: float, beta2: float, lr: float, eps: float,
                               inv_sqrt_bias_correction_2: float, inv_bias_correction_1: float,
                               weight_decay_factor: float, stochastic_round: bool = False, rng_seed: int = 0,
                               step_scalars: Optional[torch.Tensor] = None,
                               codebook_lut: Optional[torch.Tensor] = None,
                               seed_dev: Optional[torch.Tensor] = None) -> None:
    _block_update(p, grad_view, m_sign, m_magnitude, vmean, codebook, packed_indices, beta1,
                  beta2, lr, eps, inv_sqrt_bias_correction_2, inv_bias_correction_1,
                  weight_decay_factor, stochastic_round, rng_seed, step_scalars, seed_dev,
                  "automatic_gefen_fused_update_v2_full_cuda")


def _quantized_momentum_update_impl(grad_view: torch.Tensor, m_sign: torch.Tensor,
                                    m_magnitude: torch.Tensor, codebook: torch.Tensor,
                                    momentum_out: torch.Tensor, beta1: float,
                                    stochastic_round: bool = False, rng_seed: int = 0,
                                    seed_dev: Optional[torch.Tensor] = None,
                                    codebook_lut: Optional[torch.Tensor] = None,
                                    nesterov: bool = False) -> None:
    for name, t in (("m_sign", m_sign), ("m_magnitude", m_magnitude),
                    ("codebook", codebook), ("momentum_out", momentum_out)):
        if t.device != grad_view.device:
            raise ValueError("{} device {} must match grad_view device {}.".format(
                name, t.device, grad_view.device))
    if momentum_out.dtype != grad_view.dtype or momentum_out.numel() != grad_view.numel():
        raise ValueError("momentum_out must match grad_view dtype and numel")
    if not momentum_out.is_contiguous():
        raise ValueError("momentum_out must be contiguous")
    if grad_view.dtype == torch.float64:
        raise NotImplementedError("Gefen momentum kernel is not implemented for 'Double'")
    if grad_view.numel() == 0:
        return
    period = _period_of(grad_view, m_magnitude)
    grad_c = grad_view if grad_view.is_contiguous() else grad_view.contiguous()
    _, sd = _scalar_ptrs(None, seed_dev)
    qt = quant_table(codebook, grad_view.dtype)
    ws = workspace_for(m_magnitude, _native.WS_MOMENTUM, 0, 0, m_magnitude.numel())
    lib = _native.load()
    _native.check(lib.gefenx_quantized_momentum_update(
        grad_c.data_ptr(), _dtype_code(grad_view.dtype), grad_view.numel(), period,
        m_sign.data_ptr(), m_magnitude.data_ptr(), qt.data_ptr(), momentum_out.data_ptr(),
        float(beta1), 1 if stochastic_round else 0, int(rng_seed), sd, 1 if nesterov else 0,
        ws.data_ptr(), ws.numel(), _stream(grad_view.device)),
        "gefen_quantized_momentum_update_cuda")


def _momentum_apply_impl(p: torch.Tensor, grad_view: torch.Tensor, m_sign: torch.Tensor,
                         m_magnitude: torch.Tensor, stepsize: torch.Tensor, codebook: torch.Tensor,
                         packed_indices: bool, beta1: float, lr: float, what: str) -> None:
    _check_common(p, grad_view, m_sign, m_magnitude, codebook, packed_indices)
    if stepsize.device != p.device:
        raise ValueError("stepsize device {} must match p device {}.".format(stepsize.device, p.device))
    if stepsize.dtype != torch.float32:
        raise ValueError("stepsize must be float32, got {}.".format(stepsize.dtype))
    if p.numel() == 0:
        return
    if stepsize.numel() != m_magnitude.numel():
        raise ValueError("stepsize must hold one entry per block ({}), got {}".format(
            m_magnitude.numel(), stepsize.numel()))
    if not p.is_contiguous():
        raise ValueError("p must be contiguous")
    period = _period_of(grad_view, m_magnitude)
    grad_c = grad_view if grad_view.is_contiguous() else grad_view.contiguous()
    step_c = stepsize if stepsize.is_contiguous() else stepsize.contiguous()
    qt = quant_table(codebook, p.dtype)
    ws = workspace_for(m_magnitude, _native.WS_BLOCK, 1, p.numel(), m_magnitude.numel())
    _native.check(_native.load().gefenx_momentum_apply(
        p.data_ptr(), grad_c.data_ptr(), _dtype_code(p.dtype), p.numel(), period, m_sign.data_ptr(),
        m_magnitude.data_ptr(), step_c.data_ptr(), qt.data_ptr(), float(beta1), float(lr), ws.data_ptr(),
        ws.numel(), _stream(p.device)), what)


def automatic_gefen_fused_update_cuda(p: torch.Tensor, grad_view: torch.Tensor, m_sign: torch.Tensor,
                                      m_magnitude: torch.Tensor, stepsize: torch.Tensor,
                                      codebook: torch.Tensor, packed_indices: bool, beta1: float,
                                      lr: float, *, use_v2: Optional[bool] = None) -> None:
    """Legacy partial update (reference :202-265): requantise the momentum and
    apply p -= c[idx'] * mag' * stepsize[b] * lr with the caller's per-block
    stepsize (no second moment, no weight decay).  `use_v2` picks between the
    reference's two kernels, which compute the same step; both routes reach
    one C-ABI function here (gefenx_momentum_apply)."""
    _momentum_apply_impl(p, grad_view, m_sign, m_magnitude, stepsize, codebook, packed_indices, beta1, lr,
                         "automatic_gefen_fused_update_cuda")


def _factored_v_ema_impl(v_row: torch.Tensor, v_col: torch.Tensor, row_sq: torch.Tensor,
                         col_sq: torch.Tensor, beta2: float) -> None:
    """Standalone factored EMA (reference binding :114-120, kernel
    :2792-2850): v_row = v_row*beta2 + (row_sq/cols)*(1-beta2) and the same
    for v_col with rows, as the GPU aten chain rounds it."""
    tensors = (("v_row", v_row), ("v_col", v_col), ("row_sq", row_sq), ("col_sq", col_sq))
    for name, t in tensors:
        if t.device.type != "cuda":
            raise ValueError("Expected all tensors to be on CUDA ({} is on {}).".format(name, t.device))
        if t.device != v_row.device:
            raise ValueError("Expected all tensors on the same device.")
        if not t.is_contiguous():
            raise ValueError("Expected all tensors to be contiguous.")
        if t.dtype != torch.float32:
            raise ValueError("Expected all tensors to have dtype float32.")
    rows, cols = v_row.numel(), v_col.numel()
    if row_sq.numel() != rows or col_sq.numel() != cols:
        raise ValueError("Expected row_sq/col_sq numel to match v_row/v_col.")
    _native.check(_native.load().gefenx_factored_v_ema(
        v_row.data_ptr(), v_col.data_ptr(), row_sq.data_ptr(), col_sq.data_ptr(), rows, cols, float(beta2),
        _stream(v_row.device)), "gefen_factored_v_ema_cuda")


def _check_lut(lut: Optional[torch.Tensor], codebook: torch.Tensor) -> None:
    """The reference binding's `lut` argument: int16 with >= 2 entries on the
    codebook's device, or empty (= full search).  The quantisation table is
    derived from the codebook itself, so a valid LUT changes nothing."""
    if lut is None or lut.numel() == 0:
        return
    if lut.dtype != torch.int16 or lut.numel() < 2:
        raise ValueError("codebook LUT must be int16 with >= 2 entries (or empty)")
    if lut.device != codebook.device:
        raise ValueError("codebook LUT device {} must match codebook device {}.".format(lut.device, codebook.device))


class _Extension:
    """The object `_load_extension()` returns: the reference's pybind module
    surface (kernels/automatic_gefen_fused_binding.cpp:122-256) -- the same
    function names and positional argument order, `lut` included -- over the
    C ABI.  The reference's tests call these names directly."""

    @staticmethod
    def automatic_gefen_fused_update_cuda(p, grad_view, m_sign, m_magnitude, stepsize, codebook, packed_indices,
                                          beta1, lr):
        _momentum_apply_impl(p, grad_view, m_sign, m_magnitude, stepsize, codebook, packed_indices, beta1, lr,
                             "automatic_gefen_fused_update_cuda")

    @staticmethod
    def automatic_gefen_fused_update_v2_cuda(p, grad_view, m_sign, m_magnitude, stepsize, codebook,
                                             packed_indices, beta1, lr):
        _momentum_apply_impl(p, grad_view, m_sign, m_magnitude, stepsize, codebook, packed_indices, beta1, lr,
                             "automatic_gefen_fused_update_v2_cuda")

    @staticmethod
    def automatic_gefen_fused_full_update_cuda(p, grad_view, m_sign, m_magnitude, vmean, codebook, lut,
                                               packed_indices, beta1, beta2, lr, eps, inv_sqrt_bias_correction_2,
                                               inv_bias_correction_1, weight_decay_factor, stochastic_round=False,
                                               rng_seed=0, step_scalars=None, seed_dev=None):
        _check_lut(lut, codebook)
        _block_update(p, grad_view, m_sign, m_magnitude, vmean, codebook, packed_indices, beta1, beta2, lr, eps,
                      inv_sqrt_bias_correction_2, inv_bias_correction_1, weight_decay_factor, stochastic_round,
                      rng_seed, step_scalars, seed_dev, "automatic_gefen_fused_full_update_cuda")

    @staticmethod
    def automatic_gefen_fused_update_v2_full_cuda(p, grad_view, m_sign, m_magnitude, vmean, codebook, lut,
                                                  packed_indices, beta1, beta2, lr, eps,
                                                  inv_sqrt_bias_correction_2, inv_bias_correction_1,
                                                  weight_decay_factor, stochastic_round=False, rng_seed=0,
                                                  step_scalars=None, seed_dev=None):
        _check_lut(lut, codebook)
        _block_update(p, grad_view, m_sign, m_magnitude, vmean, codebook, packed_indices, beta1, beta2, lr, eps,
                      inv_sqrt_bias_correction_2, inv_bias_correction_1, weight_decay_factor, stochastic_round,
                      rng_seed, step_scalars, seed_dev, "automatic_gefen_fused_update_v2_full_cuda")

    @staticmethod
    def gefen_quantized_momentum_update_cuda(grad_view, m_sign, m_magnitude, codebook, lut, momentum_out, beta1,
                                             stochastic_round, rng_seed, seed_dev, nesterov):
        _check_lut(lut, codebook)
        _quantized_momentum_update_impl(grad_view, m_sign, m_magnitude, codebook, momentum_out, beta1,
                                        stochastic_round, rng_seed, seed_dev, None, nesterov)

    @staticmethod
    def gefen_factored_update_cuda(p, grad_view, m_sign, m_magnitude, v_row, v_col, codebook, lut, cols, beta1,
                                   beta2, lr, eps, inv_bias_correction_2, inv_bias_correction_1,
                                   weight_decay_factor, stochastic_round=False, rng_seed=0, step_scalars=None,
                                   seed_dev=None):
        _check_lut(lut, codebook)
        _factored_update_impl(p, grad_view, m_sign, m_magnitude, v_row, v_col, codebook, cols, beta1, beta2, lr,
                              eps, inv_bias_correction_2, inv_bias_correction_1, weight_decay_factor,
                              stochastic_round, rng_seed, step_scalars, None, seed_dev)

    @staticmethod
    def gefen_factored_v_ema_cuda(v_row, v_col, row_sq, col_sq, beta2):
        _factored_v_ema_impl(v_row, v_col, row_sq, col_sq, beta2)


_EXTENSION_MODULE: Optional[_Extension] = None


def _load_extension() -> _Extension:
    """Reference :124-136: the extension module, loading the gfx950 library
    on first use (raises if it is missing or does not load)."""
    global _EXTENSION_MODULE
    if _EXTENSION_MODULE is None:
        _native.load()
        _EXTENSION_MODULE = _Extension()
    return _EXTENSION_MODULE


# ---------------------------------------------------------------- compile surface

def _compile_op_fake(*args, **kwargs) -> None:
    """The ops return nothing and only mutate their declared arguments."""
    return None


def _register_compile_ops() -> bool:
    """torch.library custom ops ``gefen::fused_full_update``,
    ``gefen::factored_update``, ``gefen::quantized_momentum_update`` and
    ``gefen::fused_update_v2_full`` (reference kernels/automatic_gefen_fused.py:
    440-509), each running the C-ABI implementation below, so a traced
    optimizer step keeps the kernel calls in its graph as opaque mutating ops
    instead of breaking the graph at every call.  The public wrappers route
    through them only while tracing and only on the capturable entry (device
    step scalars and a codebook LUT given); eager calls run the same
    implementation directly.  These kernels never rebind a state tensor's
    storage (magnitudes are written in place), so the in-place mutation
    contract holds on every path.  A registration failure leaves the eager
    path intact and warns once."""
    custom_op = getattr(torch.library, "custom_op", None)
    if custom_op is None:
        return False
    try:
        for name, fn, mutates in (
                ("fused_full_update", _fused_full_update_impl, ("p", "m_sign", "m_magnitude", "vmean")),
                ("factored_update", _factored_update_impl, ("p", "m_sign", "m_magnitude", "v_row", "v_col")),
                ("quantized_momentum_update", _quantized_momentum_update_impl,
                 ("m_sign", "m_magnitude", "momentum_out")),
                ("fused_update_v2_full", _fused_update_v2_full_impl, ("p", "m_sign", "m_magnitude", "vmean"))):
            opdef = custom_op("gefen::" + name, fn, mutates_args=mutates)
            opdef.register_fake(_compile_op_fake)
    except Exception as exc:  # noqa: BLE001 -- degrade to the eager path, loudly
        warnings.warn("gefen: torch.library custom-op registration failed ({}: {}); torch.compile(step) "
                      "will graph-break at each fused kernel call".format(type(exc).__name__, exc),
                      RuntimeWarning, stacklevel=2)
        return False
    return True


_COMPILE_OPS_REGISTERED = _register_compile_ops()


def _tracing() -> bool:
    return _COMPILE_OPS_REGISTERED and torch.compiler.is_compiling()


def automatic_gefen_fused_full_update_cuda(p, grad_view, m_sign, m_magnitude, vmean, codebook,
                                           packed_indices, beta1, beta2, lr, eps,
                                           inv_sqrt_bias_correction_2, inv_bias_correction_1,
                                           weight_decay_factor, stochastic_round=False,
                                           rng_seed=0, step_scalars=None, codebook_lut=None,
                                           seed_dev=None) -> None:
    """Block-vmean fused update (reference :511-579, v1-full).  step_scalars:
    fp32 device [lr, 1/sqrt(bc2), 1/bc1, wd factor] read by the kernel
    (capturable); seed_dev: int64 device seed for stochastic rounding."""
    args = (p, grad_view, m_sign, m_magnitude, vmean, codebook, packed_indices, beta1, beta2, lr, eps,
            inv_sqrt_bias_correction_2, inv_bias_correction_1, weight_decay_factor, stochastic_round,
            rng_seed, step_scalars, codebook_lut, seed_dev)
    if step_scalars is not None and codebook_lut is not None and _tracing():
        torch.ops.gefen.fused_full_update(*args)
        return
    _fused_full_update_impl(*args)


def automatic_gefen_fused_update_v2_full_cuda(p, grad_view, m_sign, m_magnitude, vmean, codebook,
                                              packed_indices, beta1, beta2, lr, eps,
                                              inv_sqrt_bias_correction_2, inv_bias_correction_1,
                                              weight_decay_factor, stochastic_round=False,
                                              rng_seed=0, step_scalars=None, codebook_lut=None,
                                              seed_dev=None) -> None:
    """Block-vmean fused update (reference :712-771, v2-full): same kernels."""
    args = (p, grad_view, m_sign, m_magnitude, vmean, codebook, packed_indices, beta1, beta2, lr, eps,
            inv_sqrt_bias_correction_2, inv_bias_correction_1, weight_decay_factor, stochastic_round,
            rng_seed, step_scalars, codebook_lut, seed_dev)
    if step_scalars is not None and codebook_lut is not None and _tracing():
        torch.ops.gefen.fused_update_v2_full(*args)
        return
    _fused_update_v2_full_impl(*args)


def gefen_factored_update_cuda(p, grad_view, m_sign, m_magnitude, v_row, v_col, codebook, cols,
                               beta1, beta2, lr, eps, inv_bias_correction_2,
                               inv_bias_correction_1, weight_decay_factor,
                               stochastic_round=False, rng_seed=0, step_scalars=None,
                               codebook_lut=None, seed_dev=None) -> None:
    """Factored second-moment fused update of one 2D param (reference :581-650).
    p may be a strided (e.g. transposed) view: the kernel walks it in logical
    row-major order, so no contiguous copy is made.  step_scalars (capturable):
    fp32 device [lr, 1/bc2, 1/bc1, wd factor]."""
    args = (p, grad_view, m_sign, m_magnitude, v_row, v_col, codebook, cols, beta1, beta2, lr, eps,
            inv_bias_correction_2, inv_bias_correction_1, weight_decay_factor, stochastic_round, rng_seed,
            step_scalars, codebook_lut, seed_dev)
    if step_scalars is not None and codebook_lut is not None and _tracing():
        torch.ops.gefen.factored_update(*args)
        return
    _factored_update_impl(*args)


def gefen_quantized_momentum_update_cuda(grad_view, m_sign, m_magnitude, codebook, momentum_out,
                                         beta1, stochastic_round=False, rng_seed=0,
                                         seed_dev=None, codebook_lut=None,
                                         nesterov=False) -> None:
    """Muon momentum: advance the quantised EMA and emit the dense momentum
    (reference :652-710).  Magnitudes are written in place, so the op is
    traceable on both the capturable and the default path."""
    args = (grad_view, m_sign, m_magnitude, codebook, momentum_out, beta1, stochastic_round, rng_seed,
            seed_dev, codebook_lut, nesterov)
    if codebook_lut is not None and _tracing():
        torch.ops.gefen.quantized_momentum_update(*args)
        return
    _quantized_momentum_update_impl(*args)
