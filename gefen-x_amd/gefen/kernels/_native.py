"""ctypes binding of the MI355X C ABI (include/gefenx.h, libgefenx.so).

The shared library is built in-tree by ``__graft_entry__.build()`` (hipcc,
gfx950) into this directory.  Loading never falls back to anything: a missing
or broken library raises ``NativeLibraryError`` (a RuntimeError), which the
optimizer treats exactly like the reference treats a failed JIT build
(gefen.py:1566-1592).

Status codes map to the reference's exception types (pybind11 translation of
std::invalid_argument, the Double dispatch rejection and launch failures):
GEFENX_EINVAL -> ValueError, GEFENX_EDTYPE -> NotImplementedError, anything
else -> RuntimeError.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libgefenx.so"
LIB_PATH = os.path.join(_HERE, LIB_NAME)

GEFENX_OK = 0
GEFENX_EINVAL = -1
GEFENX_EDTYPE = -2
GEFENX_ELAUNCH = -3
GEFENX_ENOMEM = -4

# GEFENX_ABI_VERSION this binding is written against (include/gefenx.h):
# the struct layouts and workspace sizes below follow it.
ABI_VERSION = 3

DT_F32, DT_F16, DT_BF16, DT_F64 = 0, 1, 2, 3
WS_FACTORED, WS_BLOCK, WS_MOMENTUM = 0, 1, 2


class NativeLibraryError(RuntimeError):
    """The gfx950 shared library is missing or failed to load."""


class TensorDesc(ctypes.Structure):
    """Mirror of ``gefenx_tensor_desc`` (include/gefenx.h)."""

    _fields_ = [
        ("p", ctypes.c_void_p), ("grad", ctypes.c_void_p),
        ("m_codebook", ctypes.c_void_p), ("m_magnitude", ctypes.c_void_p),
        ("v0", ctypes.c_void_p), ("v1", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
        ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
        ("ps0", ctypes.c_int64), ("ps1", ctypes.c_int64),
        ("gs0", ctypes.c_int64), ("gs1", ctypes.c_int64),
        ("period", ctypes.c_int64),
        ("dtype", ctypes.c_int32), ("factored", ctypes.c_int32),
        ("lr", ctypes.c_float), ("eps", ctypes.c_float), ("inv_bc2", ctypes.c_float),
        ("inv_bc1", ctypes.c_float), ("wd_factor", ctypes.c_float),
        ("lerp_w", ctypes.c_float), ("beta2", ctypes.c_float), ("alpha2", ctypes.c_float),
        ("bc2_div", ctypes.c_float),
    ]


class CaptDesc(ctypes.Structure):
    """Mirror of ``gefenx_capt_desc`` (include/gefenx.h)."""

    _fields_ = [
        ("step", ctypes.c_void_p), ("bc2_step", ctypes.c_void_p), ("scalars", ctypes.c_void_p),
        ("lr_dev", ctypes.c_void_p), ("lr", ctypes.c_double), ("weight_decay", ctypes.c_double),
        ("beta1", ctypes.c_double), ("beta2", ctypes.c_double),
        ("lr_dtype", ctypes.c_int32), ("sqrt_bc2", ctypes.c_int32),
    ]


class MuonItem(ctypes.Structure):
    """Mirror of ``gefenx_muon_item`` (include/gefenx.h)."""

    _fields_ = [
        ("grad", ctypes.c_void_p), ("grad_stride0", ctypes.c_int64), ("grad_stride1", ctypes.c_int64),
        ("m_codebook", ctypes.c_void_p), ("m_magnitude", ctypes.c_void_p), ("period", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_size_t),
        ("param", ctypes.c_void_p), ("param_stride0", ctypes.c_int64), ("param_stride1", ctypes.c_int64),
        ("normuon_v", ctypes.c_void_p), ("normuon_step_dev", ctypes.c_void_p), ("normuon_step", ctypes.c_int64),
        ("step_scalars", ctypes.c_void_p),
    ]


_lock = threading.Lock()
_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_D = ctypes.c_double
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); every symbol here is declared in include/gefenx.h
SIGNATURES = {
    "gefenx_abi_version": (_I, []),
    "gefenx_last_error": (ctypes.c_char_p, []),
    "gefenx_qtable_bytes": (_SZ, []),
    "gefenx_qtable_build": (_I, [_P, _I, _I, _P]),
    "gefenx_search_lut": (_I, [_P, _I, _I, _P]),
    "gefenx_workspace_bytes": (_SZ, [_I, _I64, _I64, _I64]),
    "gefenx_factored_update": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64,
                                    _P, _P, _P, _P, _I64, _P,
                                    _D, _D, _D, _D, _D, _D, _D, _I, _I64, _P, _P,
                                    _P, _SZ, _P]),
    "gefenx_factored_update_noalloc": (_I, [_P, _P, _I, _I64, _I64, _I64, _I64, _I64, _I64,
                                            _P, _P, _P, _P, _I64, _P,
                                            _D, _D, _D, _D, _D, _D, _D, _I, _I64, _P, _P, _P]),
    "gefenx_momentum_apply": (_I, [_P, _P, _I, _I64, _I64, _P, _P, _P, _P, _D, _D, _P, _SZ, _P]),
    "gefenx_block_update": (_I, [_P, _P, _I, _I64, _I64, _P, _P, _P, _P,
                                 _D, _D, _D, _D, _D, _D, _D, _I, _I64, _P, _P,
                                 _P, _SZ, _P]),
    "gefenx_quantized_momentum_update": (_I, [_P, _I, _I64, _I64, _P, _P, _P, _P, _D, _I,
                                              _I64, _P, _I, _P, _SZ, _P]),
    "gefenx_factored_v_ema": (_I, [_P, _P, _P, _P, _I64, _I64, _D, _P]),
    "gefenx_vmean_update": (_I, [_P, _P, _I, _I64, _I64, _D, _P]),
    "gefenx_exact_histogram": (_I, [_P, _I, _I64, _I64, _P, _I, _P]),
    "gefenx_block_variance_errors": (_I, [_P, _I, _I64, _P, _I, _P, _P]),
    "gefenx_block_variance_errors_ex": (_I, [_P, _I, _I64, _P, _I, _I, _P, _P]),
    "gefenx_exact_dp": (_I, [_P, _P, _I, _I, _I, _P]),
    "gefenx_exact_dp_device": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "gefenx_multi_tensor_step": (_I, [_P, _I, _P, _I, _I64, _P, _SZ, _P]),
    "gefenx_multi_tensor_scratch_bytes": (_SZ, [_I]),
    "gefenx_mt_plan_create": (_I, [_P, _I, _P, _P, _I, _I64, _P, _I, _P, _P]),
    "gefenx_mt_plan_device_bytes": (_SZ, [_P]),
    "gefenx_mt_plan_launch": (_I, [_P, _P, _SZ, _P]),
    "gefenx_mt_plan_destroy": (None, [_P]),
    "gefenx_ns_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "gefenx_newton_schulz": (_I, [_P, _I, _P, _I64, _I64, _I64, _P, _I, _D, _P, _SZ, _P]),
    "gefenx_normuon_workspace_bytes": (_SZ, [_I64]),
    "gefenx_normuon_scale": (_I, [_P, _I64, _I64, _P, _D, _I64, _D, _P, _P, _SZ, _P, _P]),
    "gefenx_muon_apply": (_I, [_P, _I, _P, _P, _I64, _I64, _D, _D, _D, _P, _D, _P]),
    "gefenx_muon_momentum_batch": (_I, [_P, _I, _I, _I64, _I64, _P, _P, _D, _I, _I64, _P, _I, _P]),
    "gefenx_normuon_batch_workspace_bytes": (_SZ, [_I, _I64]),
    "gefenx_normuon_scale_batch": (_I, [_P, _I, _P, _I64, _I64, _D, _D, _P, _P, _SZ, _P]),
    "gefenx_muon_apply_batch": (_I, [_P, _I, _I, _P, _P, _I64, _I64, _D, _D, _D, _D, _P, _P]),
    "gefenx_muon_cautious_count_batch": (_I, [_P, _I, _I, _P, _P, _I64, _I64, _P, _P]),
    "gefenx_gemm_nt_bf16": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _F, _F, _P]),
    "gefenx_profile_enable": (_I, [_I]),
    "gefenx_profile_read": (_I, [_I, _P, _P, _P, _P]),
    "gefenx_profile_reset": (_I, []),
}

K_STATS, K_FINALIZE, K_APPLY, K_MOMENTUM, K_NS_GEMM, K_BLOCK_STATS, K_BLOCK_APPLY = 0, 1, 2, 3, 4, 5, 6


def profile_read(kind: int):
    """(total_ms, launches, algorithmic_bytes, algorithmic_flops) of one kernel kind."""
    ms = ctypes.c_double(0.0)
    n = ctypes.c_int64(0)
    b = ctypes.c_double(0.0)
    f = ctypes.c_double(0.0)
    check(load().gefenx_profile_read(kind, ctypes.byref(ms), ctypes.byref(n), ctypes.byref(b),
                                     ctypes.byref(f)), "profile read")
    return ms.value, n.value, b.value, f.value


def load(path: str = LIB_PATH):
    """Load (once) and return the ctypes library; raises NativeLibraryError."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise NativeLibraryError(
                "gefen native library not built: {} is missing (run "
                "__graft_entry__.build())".format(path))
        try:
            lib = ctypes.CDLL(path)
        except OSError as exc:
            raise NativeLibraryError("failed to load {}: {}".format(path, exc)) from exc
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as exc:
                raise NativeLibraryError("{} does not export {}".format(path, name)) from exc
            fn.restype = res
            fn.argtypes = args
        built = lib.gefenx_abi_version()
        if built != ABI_VERSION:
            raise NativeLibraryError(
                "{} implements gefenx ABI version {}, this binding needs {} (rebuild with "
                "__graft_entry__.build())".format(path, built, ABI_VERSION))
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().gefenx_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(status: int, what: str = "") -> None:
    """Map a gefenx status code to the reference's Python exception types."""
    if status == GEFENX_OK:
        return
    msg = last_error() or what
    if status == GEFENX_EINVAL:
        raise ValueError(msg)
    if status == GEFENX_EDTYPE:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)
