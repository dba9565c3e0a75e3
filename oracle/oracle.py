"""CPU oracle for the Gefen optimizer step -- TEST INFRASTRUCTURE ONLY.

Thin numpy/ctypes front end over ``oracle/gefen_oracle.c`` plus the pieces of
the reference that are plain numpy/float64 host math (period search, exact-DP
driver).  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this module; the product path never does.

Every function cites the reference file:line it restates (paths relative to the
reference repo root, ``src/gefen/`` omitted).

Parity status of each function (how it is pinned):
  nearest_indices      closed form + reference golden vectors (tests/golden)
  search_lut           closed form + "LUT search == full search" invariant
  momentum_update      reference golden vectors of the CPU step
  factored_step        reference golden vectors (config-1 shaped trajectory)
  block_step           reference golden vectors (bf16/fp16/fp32, several P)
  exact_histogram      reference golden vectors + integer order-freedom
  exact_dp             reference golden vectors (pure-Python DP) + brute force
  find_period          reference golden vectors + closed-form rule tests
  sr_quantize          published SplitMix64 outputs, unbiasedness, bracket and
                       endpoint cases (tests/test_oracle_sr.py)
  vmean_update         reference golden block-step trajectories (through
                       block_step) and the decomposition block_step = vmean_update
                       + stepsize + partial_update (tests/test_oracle_boundary.py)
  partial_update       the same decomposition against the pinned block_step
  factored_v_ema       closed-form special cases (beta2 = 0, zero sums, power-of-two
                       n) and agreement with factored_step's EMA where the
                       reciprocal multiply is exact
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from typing import Iterable, List, Optional, Sequence, Tuple

import numpy as np

F32, F16, BF16 = 0, 1, 2
_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libgefen_oracle.so")
_LIB = None


def build() -> str:
    """Compile the C oracle (``oracle/Makefile``); returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def _lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    P = ctypes.c_void_p
    i64 = ctypes.c_int64
    d = ctypes.c_double
    i = ctypes.c_int
    f = ctypes.c_float
    lib.orc_round.restype = f
    lib.orc_round.argtypes = [f, i]
    lib.orc_round_array.argtypes = [P, i64, i]
    lib.orc_nearest_array.argtypes = [P, i, P, i64, P]
    lib.orc_search_lut.argtypes = [P, i, i, P]
    lib.orc_momentum_update.argtypes = [P, P, P, i64, i64, P, i, i, f, P, P]
    lib.orc_muon_momentum.argtypes = [P, P, P, i64, i64, P, i, i, d, i, P]
    lib.orc_factored_step.argtypes = [P, P, P, P, P, P, i64, i64, i64, P, i, i,
                                      d, d, d, d, d, d, d]
    lib.orc_vmean_update.argtypes = [P, P, i64, i64, i, d]
    lib.orc_block_step.argtypes = [P, P, P, P, P, i64, i64, P, i, i,
                                   d, d, d, d, d, d, d]
    lib.orc_exact_histogram.argtypes = [P, i64, i64, i, P]
    lib.orc_exact_histogram_form.argtypes = [P, i64, i64, i, P, i]
    lib.orc_exact_dp_kernel.restype = i
    lib.orc_exact_dp_kernel.argtypes = [P, P, P, i, i, i, P]
    lib.orc_sr_uniform.restype = f
    lib.orc_sr_uniform.argtypes = [ctypes.c_uint64, i64]
    lib.orc_sr_quantize.restype = ctypes.c_uint8
    lib.orc_sr_quantize.argtypes = [P, i, f, ctypes.c_uint64, i64]
    lib.orc_set_rounding.argtypes = [i, ctypes.c_uint64]
    lib.orc_set_threads.argtypes = [i]
    lib.orc_set_threads(1)
    lib.orc_factored_v_ema.argtypes = [P, P, i64, i64, d]
    lib.orc_partial_update.argtypes = [P, P, P, P, P, i64, i64, P, i, i, d, d]
    _LIB = lib
    return lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def set_threads(n: int) -> None:
    """Host threads of the step functions; results are bit-identical for
    every thread count (the parallel loops keep each element's order)."""
    _lib().orc_set_threads(int(n))


def round_dtype(x: np.ndarray, dtype: int) -> np.ndarray:
    """Round fp32 values through bf16/fp16 (RNE) and back to fp32."""
    out = _f32(x).copy()
    _lib().orc_round_array(_ptr(out), out.size, dtype)
    return out


# ------------------------------------------------------------------ search


def nearest_indices(codebook, values) -> np.ndarray:
    """gefen_nearest_codebook_indices: gefen.py:288-334."""
    cb = _f32(codebook)
    x = _f32(values).reshape(-1)
    out = np.empty(x.size, dtype=np.uint8)
    _lib().orc_nearest_array(_ptr(cb), cb.size, _ptr(x), x.size, _ptr(out))
    return out.reshape(np.shape(values))


def search_lut(codebook, buckets: int = 4096) -> np.ndarray:
    """_codebook_search_lut: kernels/automatic_gefen_fused.py:81-121."""
    cb = _f32(codebook)
    lut = np.empty(buckets + 1, dtype=np.int16)
    _lib().orc_search_lut(_ptr(cb), cb.size, buckets, _ptr(lut))
    return lut


class _Rounding:
    """Requantisation of the step calls inside the block: nearest when
    `seed` is None, else the fused kernels' stochastic rounding with that
    seed (kernels/automatic_gefen_fused_kernel.cu:160-211, 273-328; element
    index = flat index in the tensor)."""

    def __init__(self, seed):
        self.seed = seed

    def __enter__(self):
        if self.seed is not None:
            _lib().orc_set_rounding(1, ctypes.c_uint64(int(self.seed) & (2**64 - 1)))

    def __exit__(self, *exc):
        if self.seed is not None:
            _lib().orc_set_rounding(0, ctypes.c_uint64(0))


def sr_uniform(seed: int, idx: int) -> float:
    """gefen_sr_uniform: kernels/automatic_gefen_fused_kernel.cu:141-151."""
    return float(_lib().orc_sr_uniform(ctypes.c_uint64(seed & (2**64 - 1)), idx))


def sr_quantize(codebook, x: float, seed: int, idx: int) -> int:
    """quantize_codebook_index (stochastic): automatic_gefen_fused_kernel.cu:160-211."""
    cb = _f32(codebook)
    return int(_lib().orc_sr_quantize(_ptr(cb), cb.size, float(x),
                                      ctypes.c_uint64(seed & (2**64 - 1)), idx))


# ---------------------------------------------------------------- momentum


def momentum_update(g, idx, mag, period, codebook, dtype, beta1, sr_seed=None):
    """Quantized-momentum recurrence: gefen.py:3438-3486.

    Returns (new_idx, new_mag, q, u) without mutating the inputs.  sr_seed:
    None (nearest rounding) or the stochastic-rounding seed.
    """
    g = _f32(g).reshape(-1)
    idx = np.ascontiguousarray(np.asarray(idx, dtype=np.uint8).reshape(-1)).copy()
    mag = _f32(mag).reshape(-1).copy()
    nb = g.size // period
    cb = _f32(codebook)
    q = np.empty_like(g)
    u = np.empty_like(g)
    with _Rounding(sr_seed):
        _lib().orc_momentum_update(_ptr(g), _ptr(idx), _ptr(mag), nb, period, _ptr(cb),
                                   cb.size, dtype, np.float32(1.0 - beta1), _ptr(q), _ptr(u))
    return idx, mag, q, u


def muon_momentum(g, idx, mag, period, codebook, dtype, beta, nesterov=True, sr_seed=None):
    """GefenMuon decomposed quantised momentum: gefen_muon.py:1136-1144, 948-974.

    Returns (new_idx, new_mag, out) without mutating the inputs; out is the
    dense momentum handed to Newton-Schulz (grad-dtype values as fp32).
    """
    g = _f32(g).reshape(-1)
    idx = np.ascontiguousarray(np.asarray(idx, dtype=np.uint8).reshape(-1)).copy()
    mag = _f32(mag).reshape(-1).copy()
    nb = g.size // period
    cb = _f32(codebook)
    out = np.empty_like(g)
    with _Rounding(sr_seed):
        _lib().orc_muon_momentum(_ptr(g), _ptr(idx), _ptr(mag), nb, period, _ptr(cb), cb.size, dtype,
                                 float(beta), 1 if nesterov else 0, _ptr(out))
    return idx, mag, out


NS_STANDARD = [(3.4445, -4.7750, 2.0315)] * 5


def bf16(x) -> np.ndarray:
    """Round to bf16 (RNE) and widen back to fp32."""
    return round_dtype(np.asarray(x, dtype=np.float32), BF16)


def newton_schulz(m, schedule=None, eps: float = 1e-7) -> np.ndarray:
    """_zeropower_via_newtonschulz: gefen_muon.py:236-291 (bf16 path).

    Every torch op of the reference returns a bf16 tensor, so each GEMM output
    and each elementwise result is rounded to bf16 once; products accumulate
    in float64 here (the reference's bf16 GEMMs accumulate in fp32), so the
    comparison carries a tolerance.
    """
    schedule = NS_STANDARD if schedule is None else [tuple(map(float, t)) for t in schedule]
    x = bf16(m)
    tall = x.shape[0] > x.shape[1]
    if tall:
        x = np.ascontiguousarray(x.T)
    norm = bf16(np.float32(np.sqrt(np.sum(x.astype(np.float64) ** 2))))
    norm = np.maximum(norm, np.float32(eps))
    x = bf16(x / bf16(norm))
    for a, b, c in schedule:
        x64 = x.astype(np.float64)
        gram = bf16((x64 @ x64.T).astype(np.float32))
        g64 = gram.astype(np.float64)
        upd = bf16((b * g64 + c * (g64 @ g64)).astype(np.float32))
        x = bf16((a * x64 + upd.astype(np.float64) @ x64).astype(np.float32))
    if tall:
        x = np.ascontiguousarray(x.T)
    return x


def normuon(ortho, v, step: int, beta2: float = 0.95, eps: float = 1e-8):
    """_normuon_normalize: gefen_muon.py:1192-1230.  Returns (new ortho (bf16
    values), new v); `step` is the normuon step after this call's increment."""
    o = bf16(ortho)
    rows, cols = o.shape
    row_norm = np.sqrt(np.sum(o.astype(np.float64) ** 2, axis=1)).astype(np.float32)
    row_sq = (row_norm * row_norm).astype(np.float32)
    v = np.asarray(v, np.float32).reshape(-1)
    alpha = np.float32((1 - beta2) / cols)
    v = (v * np.float32(beta2) + row_sq * alpha).astype(np.float32)
    bc = np.float32(1 - beta2 ** step)
    denom = (np.sqrt(v / bc) + np.float32(eps)).astype(np.float32)
    frob = np.float32(np.sqrt(np.sum(row_sq.astype(np.float64))))
    scaled = np.float32(np.sqrt(np.sum((row_norm / denom).astype(np.float64) ** 2)))
    frob_scale = frob / max(scaled, np.float32(1.17549435e-38))
    scale = bf16((frob_scale / denom).astype(np.float32))
    return bf16(o * scale[:, None]), v


def cautious_mask(update, grad, grad_dtype: int) -> np.ndarray:
    """_cautious_mask_: gefen_muon.py:396-405.  update: the bf16 update after
    Newton-Schulz (and NorMuon); grad: the raw gradient, of grad_dtype.  The
    sign test is on update * grad in torch's promoted dtype (bf16 for a bf16
    grad, else fp32); scale = fp32(numel) / fp32(max(agree, 1)), applied as a
    bf16 multiplier; a masked element keeps the sign of its zero."""
    u = bf16(update)
    g = round_dtype(np.asarray(grad, np.float32), grad_dtype)
    prod = (u * g).astype(np.float32)
    if grad_dtype == BF16:
        prod = bf16(prod)
    mask = prod > np.float32(0.0)
    agree = max(int(mask.sum()), 1)
    scale = bf16(np.array([np.float32(mask.size) / np.float32(agree)], np.float32))[0]
    return bf16((u * mask.astype(np.float32)).astype(np.float32) * scale)


def adjust_lr_ratio(fn, shape) -> float:
    """_adjust_lr_ratio: gefen_muon.py:409-419."""
    rows, cols = shape[:2]
    if fn is None or fn == "original":
        return math.sqrt(max(1, rows / cols))
    if fn == "match_rms_adamw":
        return 0.2 * math.sqrt(max(rows, cols))
    return 1.0


def muon_apply(p, update, dtype, lr: float, wd: float, adjusted_lr: float) -> np.ndarray:
    """_apply_muon_update (non-capturable, unsharded): gefen_muon.py:1286-1300.
    p <- D(p * (1 - lr*wd)) when wd > 0, then D(fma(update, alpha, p)) with
    alpha = -adjusted_lr converted to p's dtype (torch's add_ converts `alpha`
    to the tensor dtype; a `mul_` scalar stays fp32)."""
    p = np.asarray(p, np.float32)
    if wd > 0.0:
        p = round_dtype((p * np.float32(1.0 - lr * wd)).astype(np.float32), dtype)
    alpha = round_dtype(np.array([-adjusted_lr], np.float32), dtype)[0]
    upd = np.asarray(update, np.float32).astype(np.float64)
    res = (upd * np.float64(alpha) + p.astype(np.float64)).astype(np.float32)
    return round_dtype(res, dtype)


# -------------------------------------------------------------- step paths


def factored_step(p, g, idx, mag, v_row, v_col, period, codebook, dtype, *,
                  beta1, beta2, lr, eps, bc1, bc2, wd, sr_seed=None):
    """Decomposed factored step: gefen.py:2959-3018.  Returns new arrays."""
    p = _f32(p).copy()
    rows, cols = p.shape
    g = _f32(g).reshape(rows, cols)
    idx = np.ascontiguousarray(np.asarray(idx, dtype=np.uint8).reshape(-1)).copy()
    mag = _f32(mag).reshape(-1).copy()
    v_row = _f32(v_row).reshape(-1).copy()
    v_col = _f32(v_col).reshape(-1).copy()
    cb = _f32(codebook)
    with _Rounding(sr_seed):
        _lib().orc_factored_step(_ptr(p), _ptr(g), _ptr(idx), _ptr(mag), _ptr(v_row),
                                 _ptr(v_col), rows, cols, period, _ptr(cb), cb.size, dtype,
                                 beta1, beta2, lr, eps, bc1, bc2, wd)
    return p, idx, mag, v_row, v_col


def block_step(p, g, idx, mag, vmean, period, codebook, dtype, *,
               beta1, beta2, lr, eps, bc1, bc2, wd, sr_seed=None):
    """Non-fused block-vmean step: gefen.py:3776-3818 + 129-191 + 3329-3436."""
    shape = np.shape(p)
    p = _f32(p).reshape(-1).copy()
    g = _f32(g).reshape(-1)
    idx = np.ascontiguousarray(np.asarray(idx, dtype=np.uint8).reshape(-1)).copy()
    mag = _f32(mag).reshape(-1).copy()
    vmean = _f32(vmean).reshape(-1).copy()
    cb = _f32(codebook)
    with _Rounding(sr_seed):
        _lib().orc_block_step(_ptr(p), _ptr(g), _ptr(idx), _ptr(mag), _ptr(vmean), p.size,
                              period, _ptr(cb), cb.size, dtype, beta1, beta2, lr, eps,
                              bc1, bc2, wd)
    return p.reshape(shape), idx, mag, vmean


def vmean_update(vmean, g, period, dtype, beta2):
    """automatic_vmean_update(use_fused=False): gefen.py:129-191.  Returns
    the new vmean (bf16 grads square and average through bf16)."""
    g = _f32(g).reshape(-1)
    v = _f32(vmean).reshape(-1).copy()
    _lib().orc_vmean_update(_ptr(v), _ptr(g), g.size // period, period, dtype, float(beta2))
    return v


def factored_v_ema(v, sq, n, beta2):
    """gefen_factored_v_ema_cuda (kernels/automatic_gefen_fused_kernel.cu:
    1990-2042, 2792-2850): v <- fma(1-beta2, sq * RN(1/n), RN(v*beta2)), the
    rounding of the GPU aten chain v.mul_(beta2).add_(sq.div_(n), 1-beta2).
    Returns the new v."""
    v = _f32(v).reshape(-1).copy()
    sq = _f32(sq).reshape(-1)
    _lib().orc_factored_v_ema(_ptr(v), _ptr(sq), v.size, int(n), float(beta2))
    return v


def partial_update(p, g, idx, mag, stepsize, period, codebook, dtype, *, beta1, lr):
    """automatic_gefen_fused_update_cuda (kernels/automatic_gefen_fused_kernel.cu:
    331-415) on the CPU step's recurrence (gefen.py:3438-3486): momentum, then
    p <- D(p - (q * stepsize[b]) * lr).  Returns (p, idx, mag)."""
    shape = np.shape(p)
    p = _f32(p).reshape(-1).copy()
    g = _f32(g).reshape(-1)
    idx = np.ascontiguousarray(np.asarray(idx, dtype=np.uint8).reshape(-1)).copy()
    mag = _f32(mag).reshape(-1).copy()
    st = _f32(stepsize).reshape(-1)
    cb = _f32(codebook)
    _lib().orc_partial_update(_ptr(p), _ptr(g), _ptr(idx), _ptr(mag), _ptr(st), p.size, period, _ptr(cb),
                              cb.size, dtype, float(beta1), float(lr))
    return p.reshape(shape), idx, mag


# ------------------------------------------------------------ step-1 math


def exact_histogram(g, period: int, bins: int = 4096, counts=None, kernel_scale: bool = False) -> np.ndarray:
    """Block-absmax-normalised histogram: gefen.py:455-469 (bins from a
    division by f32(2/bins)); kernel_scale=True bins with a multiply by
    bins/2, as the reference's histogram kernel does
    (kernels/exact_histogram_fused_kernel.cu:66-76).  Identical for
    power-of-two bins."""
    g = _f32(g).reshape(-1)
    if counts is None:
        counts = np.zeros(bins, dtype=np.int64)
    _lib().orc_exact_histogram_form(_ptr(g), g.size, period, bins, _ptr(counts), 1 if kernel_scale else 0)
    return counts


def histogram_stats(bin_counts: np.ndarray):
    """Bin centres and active set: gefen.py:474-493 (fp32 linspace is exact)."""
    bins = bin_counts.size
    edges = np.array([-1.0 + 2.0 * k / bins for k in range(bins + 1)], dtype=np.float32)
    centers = (np.float32(0.5) * (edges[:-1] + edges[1:])).astype(np.float32)
    counts = bin_counts.astype(np.float32)
    active = counts > 0
    return centers[active], counts[active]


def exact_dp(active_centers, active_counts, num_codebooks: int = 256,
             force_endpoints: bool = True) -> np.ndarray:
    """quantization.exact_dp: quantization.py:197-253 (+ padding 59-72)."""
    centers = _f32(active_centers)
    counts = _f32(active_counts)
    if centers.size == 0:
        raise ValueError("Cannot run exact DP on an empty histogram.")
    if num_codebooks > centers.size:
        cb = np.empty(num_codebooks, dtype=np.float32)
        cb[: centers.size] = centers
        cb[centers.size:] = centers[-1]
        if force_endpoints:
            cb[0] = -1.0
            cb[-1] = 1.0
        return np.sort(cb)
    w = counts.astype(np.float64)
    c = centers.astype(np.float64)
    n = centers.size
    pw = np.zeros(n + 1)
    pwx = np.zeros(n + 1)
    pwx2 = np.zeros(n + 1)
    # torch.cumsum on CPU is a sequential inclusive scan in the input dtype
    acc_w = acc_wx = acc_wx2 = 0.0
    wx = w * c
    wx2 = w * (c * c)
    for i in range(n):
        acc_w += w[i]
        acc_wx += wx[i]
        acc_wx2 += wx2[i]
        pw[i + 1] = acc_w
        pwx[i + 1] = acc_wx
        pwx2[i + 1] = acc_wx2
    cb = np.empty(num_codebooks, dtype=np.float32)
    rc = _lib().orc_exact_dp_kernel(_ptr(pw), _ptr(pwx), _ptr(pwx2), n, num_codebooks,
                                    1 if force_endpoints else 0, _ptr(cb))
    if rc != 0:
        raise MemoryError("oracle exact DP allocation failed")
    return np.sort(cb)


def learn_codebook(grad_periods: Iterable[Tuple[np.ndarray, int]],
                   num_codebooks: int = 256) -> Optional[np.ndarray]:
    """learn_gefen_exact_codebook_from_grad_periods: gefen.py:417-517."""
    bins = num_codebooks * 16
    counts = np.zeros(bins, dtype=np.int64)
    total = 0
    for g, period in grad_periods:
        g = _f32(g).reshape(-1)
        if g.size == 0:
            continue
        exact_histogram(g, period, bins, counts)
        total += g.size
    if total == 0:
        return None
    centers, cnts = histogram_stats(counts)
    return exact_dp(centers, cnts, num_codebooks, True)


# ---------------------------------------------------------- period search


def divisors(n: int) -> List[int]:
    """partitioning.divisors: partitioning.py:50-59."""
    small, large = [], []
    for i in range(1, int(n ** 0.5) + 1):
        if n % i == 0:
            if i != n:
                small.append(i)
            if i != n // i and n // i != n:
                large.append(n // i)
    return small + large[::-1]


def _largest_divisor_at_most(n: int, cap: int) -> int:
    """partitioning.py:18-28."""
    best = 1
    for i in range(1, int(n ** 0.5) + 1):
        if n % i == 0:
            if cap >= i > best:
                best = i
            j = n // i
            if cap >= j > best:
                best = j
    return best


def memory_safe_fallback_period(n: int, shape, cap: int = 2048) -> int:
    """partitioning.memory_safe_fallback_period: partitioning.py:31-47."""
    if n < 8:
        return 1
    cands = []
    if shape is not None and len(shape) >= 2:
        inf = int(shape[-1])
        if inf >= 8 and n % inf == 0:
            cands.append(inf)
    capped = _largest_divisor_at_most(n, cap)
    if capped >= 8:
        cands.append(capped)
    if not cands:
        return 1
    return max(cands)


def block_variance_error(values64: np.ndarray, period: int) -> float:
    """average_within_block_variance_cpu: partitioning.py:62-84 (float64 numpy)."""
    blocks = values64.reshape(-1, period)
    return float(np.sqrt(blocks.var(axis=1).mean()))


def finalize_period(results: Sequence[Tuple[int, float]]) -> int:
    """_finalize_period_results: partitioning.py:237-271."""
    if not results:
        raise ValueError("Expected at least one valid period candidate.")
    scored = []
    prev = None
    for p, err in results:
        we = 1e-12 if prev is None else err - prev
        prev = err
        scored.append((p, err, we))
    _, best = min((we, p) for p, _, we in scored)
    return 1 if best < 8 else best


def find_period(grad, shape=None, *, memory_safe_fallback: bool = True,
                return_errors: bool = False):
    """find_period_by_block_variance, backend 'cpu': partitioning.py:274-313,
    fed as gefen.py:2639-2655 does (fp32 square, then float64)."""
    g = _f32(grad).reshape(-1)
    vals = (g * g).astype(np.float32).astype(np.float64)
    n = vals.size
    divs = divisors(n)
    results = [(p, block_variance_error(vals, p)) for p in divs]
    period = finalize_period(results)
    if memory_safe_fallback and period == 1:
        period = memory_safe_fallback_period(n, shape)
    if return_errors:
        return period, results
    return period


def resolve_period(grad, shape) -> int:
    """_iter_gefen_grad_periods / _resolve_automatic_period for default flags:
    gefen.py:2563-2577, 2712-2717 (numel 1 -> period 1)."""
    g = np.asarray(grad).reshape(-1)
    if g.size == 1:
        return 1
    return find_period(g, shape)
