"""GefenMuon: Muon (momentum orthogonalised by Newton-Schulz) with Gefen's
8-bit codebook-quantised momentum state.

Drop-in for the reference class (gefen_muon.py:453-3030): same constructor
arguments, param-group keys, per-parameter state (``automatic_period``,
``step``, ``m_codebook``, ``m_magnitude``, NorMuon's ``normuon_v`` /
``normuon_step``) and state_dict layout.  Per 2D parameter the step is:

  momentum     gefenx_quantized_momentum_update: advance the quantised
               momentum and emit the dense (Nesterov) momentum
               (gefen_muon.py:1064-1146);
  orthogonalise gefenx_newton_schulz on bf16 MFMA, batched over parameters of
               one shape (each matrix is computed exactly as alone, so batching
               never changes results) (gefen_muon.py:236-291, 353-393);
  normuon      gefenx_normuon_scale (gefen_muon.py:1192-1230);
  apply        gefenx_muon_apply: decoupled weight decay, then
               p += update * -lr * ratio(adjust_lr_fn) (gefen_muon.py:1234-1300).

Parameters must live on a HIP device; there is no host fallback.  Sharded
(DTensor) modes and the fp8 / compiled Newton-Schulz variants are single-GPU
no-ops here: ``sharded_mode`` is accepted and validated, ``fp8_ns`` falls back
to bf16 exactly as the reference does on hardware without its fp8 GEMM.
"""
from __future__ import annotations

import ctypes
import math
import os
import warnings
from collections import OrderedDict
from typing import Iterable, Optional, Tuple, Union

import numpy as np
import torch
import torch.nn as nn

from gefen.gefen import Gefen, _amp_gate, _stream_of
from gefen.kernels import _native
from gefen.kernels import automatic_gefen_fused as _fused

EPS = 1e-7
DEFAULT_A = 3.4445
DEFAULT_B = -4.7750
DEFAULT_C = 2.0315
DEFAULT_NS_STEPS = 5

# Tuned per-iteration coefficient schedules of the reference
# (gefen_muon.py:54-72): the same numbers, since they define the iteration.
NS_SCHEDULE_3STEP = [
    (5.0067, -14.4125, 10.6001),
    (3.7534, -6.8083, 3.3840),
    (3.2080, -4.3501, 2.0330),
]
NS_SCHEDULE_4STEP = [
    (5.4261, -15.5285, 11.2657),
    (3.0766, -4.9701, 2.1297),
    (3.0008, -6.4486, 4.3696),
    (2.8386, -4.1421, 2.5758),
]
NS_SCHEDULES = {"standard": None, "tuned3": NS_SCHEDULE_3STEP, "tuned4": NS_SCHEDULE_4STEP}

BATCHED_NS_DEFAULT_WORKSPACE_BYTES = 256 << 20
# Device memory one Newton-Schulz call may use for a shape batch (X, two X^T
# buffers, Gram and update matrices per item).
NS_WORKSPACE_BUDGET = int(os.environ.get("GEFENX_NS_WORKSPACE_BYTES", str(8 << 30)))


def _normalize_ns_schedule(ns_coefficients, ns_steps: int):
    """gefen_muon.py:189-233: a single (a, b, c) repeated ns_steps times, or an
    explicit per-iteration list (its length is the iteration count)."""
    if len(ns_coefficients) == 0:
        raise ValueError("ns_coefficients must be non-empty")
    first = ns_coefficients[0]
    if isinstance(first, (int, float)):
        if not 1 <= ns_steps < 100:
            raise ValueError(
                "ns_steps must be in [1, 100) but is: {}. 0 or a negative value would produce an EMPTY "
                "Newton-Schulz schedule (silently degrading Muon to normalized momentum SGD); 100+ is rejected "
                "for computational efficiency".format(ns_steps))
        if len(ns_coefficients) != 3:
            raise ValueError("A single coefficient set must be a tuple of exactly 3 values")
        return [tuple(float(x) for x in ns_coefficients)] * int(ns_steps)
    schedule = []
    for entry in ns_coefficients:
        if len(entry) != 3:
            raise ValueError("Each Newton-Schulz schedule entry must have exactly 3 values")
        schedule.append(tuple(float(x) for x in entry))
    if len(schedule) >= 100:
        raise ValueError("Newton-Schulz schedule length must be less than 100 for computational efficiency")
    return schedule


def _adjust_lr_ratio(adjust_lr_fn: Optional[str], param_shape) -> float:
    """gefen_muon.py:409-419."""
    rows, cols = param_shape[:2]
    if adjust_lr_fn is None or adjust_lr_fn == "original":
        return math.sqrt(max(1, rows / cols))
    if adjust_lr_fn == "match_rms_adamw":
        return 0.2 * math.sqrt(max(rows, cols))
    return 1.0


def _adjust_lr(lr, adjust_lr_fn: Optional[str], param_shape) -> float:
    """gefen_muon.py:422-428."""
    if isinstance(lr, torch.Tensor):
        lr = lr.item()
    return lr * _adjust_lr_ratio(adjust_lr_fn, param_shape)


_NS_WS: dict = {}


def _ns_workspace(device, nbytes: int) -> torch.Tensor:
    ws = _NS_WS.get(device)
    if ws is None or ws.numel() < nbytes:
        _NS_WS.pop(device, None)
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _NS_WS[device] = ws
    return ws


def _zeropower_via_newtonschulz_batched(grads: torch.Tensor, ns_coefficients, ns_steps: int,
                                        eps: float) -> torch.Tensor:
    """Newton-Schulz of a [batch, rows, cols] stack on the GPU (bf16 result in
    the input's orientation).  Reference: gefen_muon.py:353-393 (and the
    serial 236-291, which every item matches exactly here)."""
    if grads.ndim != 3:
        raise ValueError("Batched Newton-Schulz expects [batch, rows, cols]")
    schedule = _normalize_ns_schedule(ns_coefficients, ns_steps)
    if not grads.is_cuda:
        raise RuntimeError("Newton-Schulz runs on the HIP device; got a {} tensor".format(grads.device))
    x = grads if grads.is_contiguous() else grads.contiguous()
    b, r, c = x.shape
    out = torch.empty((b, r, c), dtype=torch.bfloat16, device=x.device)
    if x.numel() == 0:
        return out
    lib = _native.load()
    abc = np.ascontiguousarray(np.asarray(schedule, dtype=np.float64).reshape(-1))
    ws = _ns_workspace(x.device, int(lib.gefenx_ns_workspace_bytes(b, r, c)))
    with torch.cuda.device(x.device):
        _native.check(lib.gefenx_newton_schulz(
            x.data_ptr(), _fused._dtype_code(x.dtype), out.data_ptr(), b, r, c,
            abc.ctypes.data_as(ctypes.c_void_p), len(schedule), float(eps), ws.data_ptr(), ws.numel(),
            _stream_of(x)), "newton-schulz")
    return out


def _zeropower_via_newtonschulz(grad: torch.Tensor, ns_coefficients, ns_steps: int, eps: float,
                                use_fp8: bool = False, compile_fp8: bool = True) -> torch.Tensor:
    """gefen_muon.py:236-291 for one 2D matrix (bf16 result).  fp8 requests
    run in bf16: this build has no fp8 Newton-Schulz."""
    if len(grad.shape) != 2:
        raise ValueError("Input tensor gradient must be a 2D matrix")
    return _zeropower_via_newtonschulz_batched(grad.unsqueeze(0), ns_coefficients, ns_steps, eps)[0]


def _masked_copy_into_(update: torch.Tensor, grad, row_scale, counts) -> torch.Tensor:
    """update <- u'' in place through the Muon apply kernel applied to a
    buffer of -0: with lr 0, no weight decay and adjusted_lr -1 the apply
    computes fma(u'', 1, -0) = u'' (signed zeros included), u'' the update
    times the NorMuon row scale (row_scale) and/or cautiously masked (counts)."""
    lib = _native.load()
    rows, cols = update.shape
    u = update.contiguous()
    out_dtype = grad.dtype if grad is not None else torch.bfloat16
    out = torch.full((rows, cols), -0.0, dtype=out_dtype, device=update.device)
    item = (_native.MuonItem * 1)()
    item[0].param = out.data_ptr()
    item[0].param_stride0, item[0].param_stride1 = out.stride()
    if grad is not None:
        item[0].grad = grad.data_ptr()
        item[0].grad_stride0, item[0].grad_stride1 = grad.stride()
    with torch.cuda.device(update.device):
        _native.check(lib.gefenx_muon_apply_batch(
            item, 1, _fused._dtype_code(out_dtype), u.data_ptr(),
            None if row_scale is None else row_scale.data_ptr(), rows, cols, 0.0, 0.0, -1.0, 1.0,
            None if counts is None else counts.data_ptr(), _stream_of(update)), "muon update copy")
    update.copy_(out)
    return update


def _cautious_mask_(update: torch.Tensor, grad: torch.Tensor) -> torch.Tensor:
    """gefen_muon.py:396-405 on the GPU, in place: zero the elements of the bf16
    update whose product with grad (in torch's promoted dtype) is not > 0 and
    scale the rest by bf16(numel / max(agree, 1)).  The step itself masks
    inside its apply pass; this is the standalone form of the same kernels.
    An fp16 grad is taken as its exact fp32 copy: torch's promoted dtype for
    bf16 x fp16 is fp32, so the agreement decisions are the same, and the
    masked, scaled update (a bf16 x bf16 product, exact in fp32) is staged in
    fp32 and rounded to bf16 once, so no fp16 range or subnormal limit
    applies to it."""
    if update.dim() != 2 or update.shape != grad.shape:
        raise ValueError("_cautious_mask_ expects a 2D update and a grad of the same shape")
    if update.dtype != torch.bfloat16 or update.device.type != "cuda" or grad.device != update.device:
        raise ValueError("_cautious_mask_ expects a bf16 update and its grad on one HIP device")
    if grad.dtype == torch.float16:
        grad = grad.float()
    lib = _native.load()
    rows, cols = update.shape
    u = update.contiguous()
    item = (_native.MuonItem * 1)()
    item[0].grad = grad.data_ptr()
    item[0].grad_stride0, item[0].grad_stride1 = grad.stride()
    counts = torch.empty(1, dtype=torch.int64, device=update.device)
    with torch.cuda.device(update.device):
        _native.check(lib.gefenx_muon_cautious_count_batch(
            item, 1, _fused._dtype_code(grad.dtype), u.data_ptr(), None, rows, cols, counts.data_ptr(),
            _stream_of(update)), "cautious mask")
    return _masked_copy_into_(update, grad, None, counts)


def _swapped_param_groups_error(param: torch.Tensor) -> str:
    return ("GefenMuon only optimizes 2D parameters, got a parameter of shape {}. Route 1D (norm/bias) and "
            "embedding/head parameters to a plain Gefen/AdamW backup (GefenMuonHybrid / split_params_for_muon "
            "do this).".format(tuple(param.shape)))


class GefenMuon(Gefen):
    """Muon with Gefen's quantised momentum; arguments mirror the reference
    (gefen_muon.py:546-573)."""

    # Muon's momentum, Newton-Schulz and apply read device tensors only
    _steps_host_params = False

    def __init__(
        self,
        params: Iterable[Union[nn.Parameter, Tuple[str, nn.Parameter]]],
        lr: Union[float, torch.Tensor] = 1e-3,
        weight_decay: float = 0.1,
        momentum: float = 0.95,
        nesterov: bool = True,
        ns_coefficients=(DEFAULT_A, DEFAULT_B, DEFAULT_C),
        eps: float = EPS,
        ns_steps: int = DEFAULT_NS_STEPS,
        ns_schedule: Optional[object] = None,
        adjust_lr_fn: Optional[str] = None,
        *,
        fused: bool = True,
        sharded_mode: str = "exact",
        fp8_ns: bool = False,
        fp8_ns_compile: bool = True,
        batched_ns: bool = False,
        batched_ns_workspace_bytes: int = BATCHED_NS_DEFAULT_WORKSPACE_BYTES,
        stochastic_round: bool = False,
        deterministic: bool = False,
        normuon: bool = False,
        normuon_beta2: float = 0.95,
        normuon_eps: float = 1e-8,
        cautious: bool = False,
        capturable: bool = False,
        verbose: bool = False,
    ) -> None:
        # argument checks of gefen_muon.py:578-720
        if isinstance(lr, torch.Tensor) and lr.numel() != 1:
            raise ValueError("Tensor lr must be 1-element")
        if not 0.0 <= lr:
            raise ValueError("Learning rate should be >= 0 but is: {}".format(lr))
        if not 0.0 <= momentum < 1.0:
            raise ValueError("momentum should be in [0, 1) but is: {}".format(momentum))
        if not math.isfinite(eps) or eps <= 0.0:
            raise ValueError("eps should be finite and > 0 but is: {}. The Newton-Schulz input normalization "
                             "divides by the momentum matrix norm clamped at eps, so eps=0 turns an all-zero "
                             "momentum matrix into 0/0 = NaN".format(eps))
        if not 0.0 <= weight_decay:
            raise ValueError("weight decay should be >= 0 but is: {}".format(weight_decay))
        if adjust_lr_fn is not None and adjust_lr_fn not in ["original", "match_rms_adamw"]:
            raise ValueError("Adjust learning rate function {} is not supported".format(adjust_lr_fn))
        if sharded_mode not in ("exact", "approx", "distributed"):
            raise ValueError("sharded_mode must be 'exact', 'approx' or 'distributed' but is: {}".format(sharded_mode))
        if ns_schedule is not None:
            if isinstance(ns_schedule, str):
                if ns_schedule not in NS_SCHEDULES:
                    raise ValueError("Unknown ns_schedule {!r}; choose from {}".format(ns_schedule,
                                                                                     sorted(NS_SCHEDULES)))
                resolved = NS_SCHEDULES[ns_schedule]
            else:
                resolved = ns_schedule
            if resolved is not None:
                schedule = _normalize_ns_schedule(resolved, ns_steps)
                ns_coefficients = schedule
                ns_steps = len(schedule)
        if (len(ns_coefficients) > 0 and isinstance(ns_coefficients[0], (int, float))
                and not 1 <= ns_steps < 100):
            raise ValueError("ns_steps must be in [1, 100) but is: {}. 0 or a negative value would produce an "
                             "EMPTY Newton-Schulz schedule (silently degrading Muon to normalized momentum "
                             "SGD)".format(ns_steps))
        if not isinstance(batched_ns_workspace_bytes, int) or isinstance(batched_ns_workspace_bytes, bool):
            raise TypeError("batched_ns_workspace_bytes must be an integer")
        if batched_ns_workspace_bytes <= 0:
            raise ValueError("batched_ns_workspace_bytes must be positive")
        if not 0.0 <= normuon_beta2 < 1.0:
            raise ValueError("normuon_beta2 must be in [0, 1) but is: {}".format(normuon_beta2))
        if not math.isfinite(normuon_eps) or normuon_eps <= 0.0:
            raise ValueError("normuon_eps must be finite and > 0 but is: {}".format(normuon_eps))
        self._sharded_mode = sharded_mode
        self._fp8_ns = fp8_ns
        self._fp8_ns_compile = fp8_ns_compile
        self._batched_ns = bool(batched_ns)
        self._batched_ns_workspace_bytes = batched_ns_workspace_bytes
        self._normuon = normuon
        self._cautious = cautious
        self._muon_group_defaults = {
            "momentum": momentum, "nesterov": nesterov, "ns_coefficients": ns_coefficients,
            "ns_steps": ns_steps, "adjust_lr_fn": adjust_lr_fn, "sharded_mode": sharded_mode,
            "fp8_ns": fp8_ns, "fp8_ns_compile": fp8_ns_compile, "batched_ns": bool(batched_ns),
            "batched_ns_workspace_bytes": batched_ns_workspace_bytes, "normuon": normuon,
            "normuon_beta2": normuon_beta2, "normuon_eps": normuon_eps, "cautious": cautious,
        }
        self._muon_buffers = {}
        super().__init__(params, lr=lr, betas=(momentum, 0.0), eps=eps, weight_decay=weight_decay, fused=fused,
                         factored_v_2d=False, stochastic_round=stochastic_round, deterministic=deterministic,
                         capturable=capturable, verbose=verbose)

    def _normuon_normalize(self, state, ortho: torch.Tensor, beta2: float, eps: float) -> torch.Tensor:
        """gefen_muon.py:1192-1230 for one bf16 update, in place: the NorMuon
        row scale of gefenx_normuon_scale (normuon_v and normuon_step created
        in `state` when missing, then advanced) applied through the Muon apply
        kernel.  The step itself scales inside its apply pass."""
        if ortho.dim() != 2 or ortho.dtype != torch.bfloat16 or ortho.device.type != "cuda":
            raise ValueError("_normuon_normalize expects a 2D bf16 update on a HIP device")
        rows, cols = ortho.shape
        v = state.get("normuon_v")
        if v is None or v.shape[0] != rows:
            v = torch.zeros(rows, 1, dtype=torch.float32, device=ortho.device)
            state["normuon_v"] = v
            state["normuon_step"] = self._new_step_counter(ortho.device)
        lib = _native.load()
        u = ortho.contiguous()
        scale = torch.empty(rows, dtype=torch.bfloat16, device=ortho.device)
        ws = torch.empty(int(lib.gefenx_normuon_workspace_bytes(rows)), dtype=torch.uint8, device=ortho.device)
        step_dev = None
        if torch.is_tensor(state["normuon_step"]):
            state["normuon_step"] += 1
            step_dev = state["normuon_step"].data_ptr()
            step = 0
        else:
            state["normuon_step"] += 1
            step = int(state["normuon_step"])
        with torch.cuda.device(ortho.device):
            _native.check(lib.gefenx_normuon_scale(
                u.data_ptr(), rows, cols, v.data_ptr(), float(beta2), step, float(eps), scale.data_ptr(),
                ws.data_ptr(), ws.numel(), step_dev, _stream_of(ortho)), "normuon")
        return _masked_copy_into_(ortho, None, scale, None)

    def add_param_group(self, param_group):
        """Muon defaults filled into the group, its NorMuon options checked,
        2D parameters only (gefen_muon.py:758-800); all or nothing, as
        Gefen.add_param_group."""
        if isinstance(param_group, dict):
            param_group = dict(param_group)
            for k, v in self._muon_group_defaults.items():
                param_group.setdefault(k, v)
            if "momentum" in param_group:
                param_group["beta1"] = param_group["momentum"]
            nb2, neps = param_group["normuon_beta2"], param_group["normuon_eps"]
            if not 0.0 <= nb2 < 1.0:
                raise ValueError("normuon_beta2 must be in [0, 1) but is: {}".format(nb2))
            if not math.isfinite(neps) or neps <= 0.0:
                raise ValueError("normuon_eps must be finite and > 0 but is: {}".format(neps))
        super().add_param_group(param_group)

    def _check_group_params(self, params):
        for p in params:
            if p.ndim != 2:
                raise ValueError(_swapped_param_groups_error(p))

    # --------------------------------------------------------------- state

    def _prepare_muon_state(self, name, p, grad):
        state = self.state[p]
        if "step" not in state:
            numel = p.numel()
            if "automatic_period" in state:
                period = int(state["automatic_period"])
            elif numel == 1:
                period = 1
            else:
                period = self._resolve_automatic_period(name, p, grad)
            if numel % period != 0:
                raise ValueError("Automatic partition period {} does not divide parameter {} with numel {}".format(
                    period, name, numel))
            state["automatic_period"] = period
            state["step"] = self._new_step_counter(p.device)
            nb = numel // period
            state["m_codebook"] = torch.zeros(nb, period, dtype=torch.uint8, device=p.device)
            state["m_magnitude"] = torch.zeros(nb, 1, dtype=torch.float32, device=p.device)
        return state

    def _momentum_workspace(self, state, device):
        nb = state["m_magnitude"].numel()
        need = int(_native.load().gefenx_workspace_bytes(_native.WS_MOMENTUM, 0, 0, nb))
        ws = state.get("_gefenx_ws")
        if ws is None or ws.numel() < need or ws.device != device:
            ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)
            state["_gefenx_ws"] = ws
        return ws

    def _buffer(self, key, numel, dtype, device):
        buf = self._muon_buffers.get(key)
        if buf is None or buf.numel() < numel or buf.dtype != dtype or buf.device != device:
            buf = torch.empty(max(numel, 1), dtype=dtype, device=device)
            self._muon_buffers[key] = buf
        return buf[:numel]

    # ---------------------------------------------------------------- step

    def _validate_grads(self):
        super()._validate_grads()
        for group in self.param_groups:
            for p in group["params"]:
                if p.ndim != 2:
                    raise ValueError(_swapped_param_groups_error(p))

    def _ns_batch_limit(self, rows, cols, itemsize):
        m, n = min(rows, cols), max(rows, cols)
        per_item = 2 * (3 * m * n + 2 * m * m) + itemsize * rows * cols
        return max(1, NS_WORKSPACE_BUDGET // max(per_item, 1))

    @torch.no_grad()
    def step(self, closure=None):
        capturing = self._assert_capturable_if_capturing()
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self._validate_grads()
        # gefen_muon.py:1445-1512 (one process): overflow skips the whole step.
        if not _amp_gate(self):
            return loss
        if capturing:
            self._assert_capture_ready()
        else:
            self._maybe_refresh_gefen_codebook()
            self._ensure_gefen_global_step_devices()
        lib = _native.load()
        # shape buckets: one Newton-Schulz launch sequence per bucket chunk
        buckets = OrderedDict()
        capt_rows = {}
        for gi, group in enumerate(self.param_groups):
            for name, p in self._iter_group_params_with_names(group):
                if p.grad is None or p.numel() == 0:
                    continue
                if capturing and "step" not in self.state[p]:
                    raise RuntimeError("GefenMuon capturable: parameter {} has no state yet; its first step runs "
                                       "eagerly".format(name))
                state = self._prepare_muon_state(name, p, p.grad)
                if group.get("normuon", False):
                    v = state.get("normuon_v")
                    if v is None or v.shape[0] != p.shape[0]:
                        if capturing:
                            raise RuntimeError("GefenMuon capturable: NorMuon state of {} is created eagerly".format(
                                name))
                        state["normuon_v"] = torch.zeros(p.shape[0], 1, dtype=torch.float32, device=p.device)
                        state["normuon_step"] = self._new_step_counter(p.device)
                if self._capt_on:
                    self._capt_ready_state(state, p, capturing)
                    capt_rows.setdefault(p.device, []).append(
                        self._capt_row(group, p, state, "normuon_step" if "normuon_step" in state else None, 0))
                key = (p.device, tuple(p.shape), p.grad.dtype, gi)
                buckets.setdefault(key, []).append((group, name, p, p.grad))
        if self._capt_on:  # step counters, scalar rows, global step and seed on the device
            for device in self._capt_counters:
                self._capt_launch(device, [], [], capt_rows.get(device, []), set(), capturing)
        for (device, shape, gdtype, gi), items in buckets.items():
            group = self.param_groups[gi]
            rows, cols = shape
            schedule = _normalize_ns_schedule(group["ns_coefficients"], group["ns_steps"])
            limit = self._ns_batch_limit(rows, cols, torch.empty((), dtype=gdtype).element_size())
            for c0 in range(0, len(items), limit):
                chunk = items[c0:c0 + limit]
                self._step_chunk(lib, group, chunk, device, rows, cols, gdtype, schedule)
        self._gefen_global_step += 1
        return loss

    def _step_chunk(self, lib, group, chunk, device, rows, cols, gdtype, schedule):
        """One bucket chunk (matrices of one shape, dtype and group): batched
        momentum, batched Newton-Schulz, batched NorMuon scale and apply.
        Strided grads and parameters are read and written in place."""
        numel = rows * cols
        n = len(chunk)
        stream = torch.cuda.current_stream(device).cuda_stream
        cb = self._gefen_codebook_on(device)
        qt = _fused.quant_table(cb, gdtype)
        mom = self._buffer(("mom", device, gdtype), n * numel, gdtype, device).view(n, rows, cols)
        dcode = _fused._dtype_code(gdtype)
        normuon = bool(group.get("normuon", False))
        items = (_native.MuonItem * n)()
        seed_ptr = None
        for i, (_, name, p, grad) in enumerate(chunk):
            state = self.state[p]
            ws = self._momentum_workspace(state, device)
            scalars_ptr, seed_ptr = self._capt_pointers(state, device)
            it = items[i]
            it.grad = grad.data_ptr()
            it.grad_stride0, it.grad_stride1 = grad.stride()
            it.m_codebook = state["m_codebook"].data_ptr()
            it.m_magnitude = state["m_magnitude"].data_ptr()
            it.period = int(state["automatic_period"])
            it.workspace = ws.data_ptr()
            it.workspace_bytes = ws.numel()
            it.param = p.data_ptr()
            it.param_stride0, it.param_stride1 = p.stride()
            it.step_scalars = scalars_ptr
        with torch.cuda.device(device):
            _native.check(lib.gefenx_muon_momentum_batch(
                items, n, dcode, rows, cols, qt.data_ptr(), mom.data_ptr(), float(group["momentum"]),
                1 if self._stochastic_round else 0, self._kernel_rng_seed(), seed_ptr,
                1 if group["nesterov"] else 0, stream), "muon momentum of " + chunk[0][1])
            if not self._capt_on:
                for _, _, p, _ in chunk:
                    self.state[p]["step"] += 1
            ortho = _zeropower_via_newtonschulz_batched(mom, schedule, len(schedule), group["eps"])
            lr = 0.0 if self._capt_on else self._lr_scalar(group)  # capturable: read on the device
            wd = group["weight_decay"]
            scale_ptr = None
            if normuon:
                for i, (_, _, p, _) in enumerate(chunk):
                    state = self.state[p]
                    items[i].normuon_v = state["normuon_v"].data_ptr()
                    if self._capt_on:
                        items[i].normuon_step_dev = state["normuon_step"].data_ptr()
                    else:
                        state["normuon_step"] += 1
                        items[i].normuon_step = int(state["normuon_step"])
                scale = self._buffer(("scale", device), n * rows, torch.bfloat16, device)
                nws = self._buffer(("nws", device), int(lib.gefenx_normuon_batch_workspace_bytes(n, rows)),
                                   torch.uint8, device)
                _native.check(lib.gefenx_normuon_scale_batch(
                    items, n, ortho.data_ptr(), rows, cols, float(group["normuon_beta2"]),
                    float(group["normuon_eps"]), scale.data_ptr(), nws.data_ptr(), nws.numel(), stream),
                    "normuon of " + chunk[0][1])
                scale_ptr = scale.data_ptr()
            shape = chunk[0][2].shape
            ratio = _adjust_lr_ratio(group["adjust_lr_fn"], shape)
            adjusted = 0.0 if self._capt_on else _adjust_lr(lr, group["adjust_lr_fn"], shape)
            pcode = _fused._dtype_code(chunk[0][2].dtype)
            counts_ptr = None
            if group.get("cautious", False):
                # gefen_muon.py:1160-1161: the NorMuon-scaled update against the raw grad
                counts = self._buffer(("caut", device), n, torch.int64, device)
                _native.check(lib.gefenx_muon_cautious_count_batch(
                    items, n, pcode, ortho.data_ptr(), scale_ptr, rows, cols, counts.data_ptr(), stream),
                    "cautious mask of " + chunk[0][1])
                counts_ptr = counts.data_ptr()
            _native.check(lib.gefenx_muon_apply_batch(
                items, n, pcode, ortho.data_ptr(), scale_ptr, rows, cols, lr,
                float(wd) if wd > 0.0 else 0.0, adjusted, ratio, counts_ptr, stream), "muon apply of " + chunk[0][1])
