"""Gefen: Adam-family optimizer with 8-bit codebook-quantised momentum and a
block-shared or factored second moment (~1 byte of state per parameter).

Drop-in for the reference class (gefen.py:984-5852): same constructor
arguments, param-group layout, per-parameter state keys and state_dict format.
The step runs on MI355X through the C ABI in include/gefenx.h:

  step 1   period search per parameter (float64 block variances on the GPU,
           partitioning rule of partitioning.py:237-313) and the exact-DP
           codebook from the block-absmax-normalised 4096-bin histogram
           (gefen.py:417-517);
  2D       factored second moment (row/column EMAs, gefen.py:2784-3018);
  1D / factored_v_2d=False
           block-shared second moment (gefen.py:3488-3818).

Every step runs on the GPU, and a missing gfx950 library raises instead of
falling back to host math.  ``fused=False`` (the reference's decomposed
torch-op step and its merged small-tensor batching, gefen.py:3329-3486,
3832-4013) computes the same arithmetic, so it runs on the same kernels and
the same multi-tensor launch.  A parameter paged between devices between
steps (CPU offload) takes its state along: the state follows the parameter's
device at the next step (gefen.py:1897-1927).  A parameter that is in host
memory at step time keeps its state in host memory too, and is stepped on the
current HIP device through pinned staging (gefen/host_staging.py) with the
same kernels, bit for bit as if it lived on the device.
"""
from __future__ import annotations

import ctypes
import logging
import math
import os
import warnings
import weakref
from collections import OrderedDict
from typing import Iterable, Optional, Tuple, Union

import numpy as np
import torch
import torch.nn as nn

from gefen import host_staging
from gefen import partitioning
from gefen import quantization as quantization_module
from gefen.kernels import _native
from gefen.kernels import automatic_gefen_fused as _fused

logger = logging.getLogger(__name__)

NUM_CODEBOOKS = 256
HISTOGRAM_BINS = NUM_CODEBOOKS * 16
GEFEN_EXACT_HISTOGRAM_CHUNK = 1 << 28
_CHECKPOINT_FORMAT_VERSION = 1

# Keys of per-parameter state that exist only at run time (workspaces and the
# capturable per-step scalar row).
_RUNTIME_STATE_KEYS = ("_gefenx_ws", "_capt_scalars")

# Per-parameter state that follows a parameter paged to another device
# between steps (gefen.py:66-77, 1897-1927).
_COLOCATABLE_STATE_KEYS = ("m_codebook", "m_magnitude", "vmean", "vmean_step", "v_row", "v_col",
                           "factored_step", "step", "stepsize", "_h_buf")

# Step-like per-parameter counters: python ints, or 0-dim fp32 device tensors
# under capturable=True (gefen.py:1887-1895, 5680-5705).
_COUNTER_KEYS = ("step", "vmean_step", "factored_step", "normuon_step")

# Eager-only capturable plans kept per optimizer (plans a capture recorded are
# kept for the optimizer's lifetime).
_CAPT_PLAN_CACHE = 4

_LR_DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2, torch.float64: 3}

# numpy image of gefenx_tensor_desc (field order and offsets of the C struct)
_DESC_DTYPE = np.dtype(_native.TensorDesc)


def automatic_partition_view(flat_tensor: torch.Tensor, period: int) -> torch.Tensor:
    """gefen.py:97-115."""
    if flat_tensor.dim() != 1:
        raise ValueError("Automatic partition view expects a 1D tensor, got dim={}".format(flat_tensor.dim()))
    if period <= 0:
        raise ValueError("Automatic partition period must be positive, got {}".format(period))
    if flat_tensor.numel() % period != 0:
        raise ValueError("Automatic partition expects numel {} to be divisible by period {}".format(
            flat_tensor.numel(), period))
    return flat_tensor.view(-1, period)


def _stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _block_view_ok(p: torch.Tensor, grad: torch.Tensor, period: int) -> bool:
    """The multi-tensor launcher steps a block-path parameter in place when
    it and its grad are transposed views (strides (1, ld), ld >= rows, 16-byte
    aligned storage rows) with rows, cols and period multiples of 8; other
    non-contiguous block-path parameters take the contiguous-copy route."""
    if p.ndim != 2 or grad.ndim != 2:
        return False
    rows, cols = p.shape
    es = p.element_size()
    if rows < 2 or rows % 8 or cols % 8 or period % 8:
        return False
    for t in (p, grad):
        if t.stride(0) != 1 or t.stride(1) < rows or (t.stride(1) * es) % 16 or t.data_ptr() % 16:
            return False
    return True


# ---------------------------------------------------------------- GradScaler

def _amp_step_controls(optimizer):
    """gefen.py:614-648: read GradScaler's temporary ``found_inf`` and
    ``grad_scale`` attributes (scalar tensors or numbers) without touching any
    gradient. Returns ``(overflow, grad_scale, scale_value)``; a grad_scale
    that is non-finite or not positive is an error."""
    found_inf = getattr(optimizer, "found_inf", None)
    overflow = False
    if found_inf is not None:
        if torch.is_tensor(found_inf):
            if found_inf.numel() != 1:
                raise RuntimeError("GradScaler supplied a non-scalar found_inf tensor with shape {}".format(
                    tuple(found_inf.shape)))
            overflow = bool(found_inf.detach().item())
        else:
            overflow = bool(found_inf)
    grad_scale = getattr(optimizer, "grad_scale", None)
    scale_value = 0.0
    if torch.is_tensor(grad_scale):
        if grad_scale.numel() != 1:
            raise RuntimeError("GradScaler supplied a non-scalar grad_scale tensor with shape {}".format(
                tuple(grad_scale.shape)))
        scale_value = float(grad_scale.detach().item())
    elif grad_scale is not None:
        scale_value = float(grad_scale)
    if grad_scale is not None and (not math.isfinite(scale_value) or scale_value <= 0.0):
        raise RuntimeError("GradScaler supplied a non-finite or non-positive grad_scale")
    return overflow, grad_scale, scale_value


@torch.no_grad()
def _amp_prepare_step(optimizer) -> bool:
    """gefen.py:651-707: the optimizer side of GradScaler's native protocol.

    ``False`` on overflow: the caller returns before any codebook, state,
    counter or parameter moves. ``grad_scale is None`` means the caller already
    ran ``scaler.unscale_`` (or this is no AMP step), so gradients are left
    alone. Otherwise every gradient is multiplied in place by the fp32
    reciprocal of the scale, taken in fp64 as GradScaler.unscale_ takes it,
    with one foreach multiply per device; each gradient rounds that product in
    its own dtype."""
    overflow, grad_scale, _ = _amp_step_controls(optimizer)
    if overflow:
        return False
    if grad_scale is None:
        return True
    if torch.is_tensor(grad_scale):
        inv_scale = grad_scale.detach().double().reciprocal().float()
    else:
        inv_scale = torch.tensor(float(grad_scale), dtype=torch.float64).reciprocal().float()
    by_device = OrderedDict()
    for group in optimizer.param_groups:
        for p in group["params"]:
            if p.grad is not None:
                by_device.setdefault(p.grad.device, []).append(p.grad)
    for device, grads in by_device.items():
        torch._foreach_mul_(grads, inv_scale.to(device=device, non_blocking=True))
    return True


def _amp_native_scaling_required(optimizer) -> bool:
    """gefen.py:853-894: take the native protocol only where GradScaler's own
    unscale cannot run, which is a true fp16 gradient. fp32-master and bf16
    training keep GradScaler's ordinary path (it skips ``step`` on overflow
    itself, so schedulers see the skip). An FSDP1 FlatParameter with fp16
    gradients needs the sharded scaler's cross-rank reduction: native handling
    is declined for it with a one-time warning."""
    has_fp16_grad = False
    has_flat_param = False
    for group in optimizer.param_groups:
        for p in group["params"]:
            if getattr(p, "_is_flat_param", False):
                has_flat_param = True
            if p.grad is not None and p.grad.dtype == torch.float16:
                has_fp16_grad = True
    if has_fp16_grad and has_flat_param:
        if not getattr(optimizer, "_gefen_warned_sharded_fp16_amp", False):
            warnings.warn(
                "Gefen detected FP16 gradients on an FSDP1 FlatParameter and disabled optimizer-side AMP "
                "unscaling. Use torch.distributed.fsdp.ShardedGradScaler (or call its unscale_ before step) so "
                "non-finite detection is reduced across ranks.", RuntimeWarning, stacklevel=3)
            optimizer._gefen_warned_sharded_fp16_amp = True
        return False
    return has_fp16_grad


def _amp_gate(optimizer) -> bool:
    """True when the step should go ahead: no GradScaler controls are attached,
    or they were attached and the gradients are finite (now unscaled)."""
    if not (hasattr(optimizer, "found_inf") or hasattr(optimizer, "grad_scale")):
        return True
    return _amp_prepare_step(optimizer)


FUSE_HISTOGRAM_FOR_EXACT = True


def _exact_histogram_counts(grad_periods, bins: int):
    """gefen.py:429-468 on the histogram kernel: (int64 counts on the
    grads' device, number of elements) over (name, flat grad, period, shape)
    tuples; (None, 0) when there are none.  Chunks of
    GEFEN_EXACT_HISTOGRAM_CHUNK elements, block-aligned, so chunking is exact."""
    lib = _native.load()
    counts_dev = None
    total = 0
    for _, flat, period, _ in grad_periods:
        f = flat.reshape(-1)
        if f.device.type != "cuda":
            raise ValueError("the exact codebook histogram needs gradients on a HIP device (got {})".format(f.device))
        if not f.is_contiguous():
            f = f.contiguous()
        if counts_dev is None:
            counts_dev = torch.zeros(bins, dtype=torch.int64, device=f.device)
        elif counts_dev.device != f.device:
            raise ValueError("all parameters must live on one device")
        chunk = max(1, GEFEN_EXACT_HISTOGRAM_CHUNK // period) * period
        for start in range(0, f.numel(), chunk):
            part = f[start:start + chunk]
            _native.check(lib.gefenx_exact_histogram(
                part.data_ptr(), _fused._dtype_code(part.dtype), part.numel(), int(period),
                counts_dev.data_ptr(), bins, _stream_of(part)), "exact histogram")
        total += f.numel()
    return counts_dev, total


def learn_gefen_exact_codebook_from_grad_periods(*, grad_periods, codebook_device, num_codebooks: int,
                                                 force_endpoints: bool, verbose: bool, compute_mse_logging: bool,
                                                 use_fused_histogram: bool = FUSE_HISTOGRAM_FOR_EXACT):
    """gefen.py:417-517: the exact 1-D k-means codebook of the block-absmax
    normalised grads.  grad_periods: (name, flat grad, period, shape) tuples.
    Counts of num_codebooks * 16 bins come from the histogram kernel (int64,
    block-aligned chunks of GEFEN_EXACT_HISTOGRAM_CHUNK elements, order-free,
    so chunking is exact); the DP runs on the device of the grads.  The
    product steps on HIP devices only, so use_fused_histogram is accepted for
    the reference's signature and the grads must be device tensors.
    codebook_device None keeps the codebook on the grads' device.  Returns
    None when there are no elements."""
    del use_fused_histogram
    bins = int(num_codebooks) * 16
    counts_dev, total = _exact_histogram_counts(grad_periods, bins)
    if total == 0:
        return None
    counts = counts_dev.cpu().to(torch.float32)
    edges = torch.linspace(-1.0, 1.0, steps=bins + 1, dtype=torch.float32)
    centers = 0.5 * (edges[:-1] + edges[1:])
    active = counts > 0
    stats = {"bin_edges": edges, "bin_centers": centers, "bin_counts": counts, "active_bins": active,
             "active_centers": centers[active], "active_counts": counts[active],
             "active_sums": centers[active] * counts[active]}
    codebook = quantization_module.exact_dp(histogram_stats=stats, num_codebooks=int(num_codebooks),
                                            force_endpoints=force_endpoints, device=counts_dev.device)
    if codebook_device is not None:
        codebook = codebook.to(codebook_device)
    if verbose and compute_mse_logging:
        cb = codebook.cpu()
        ac = stats["active_centers"]
        idx = torch.searchsorted(cb, ac)
        lo, hi = (idx - 1).clamp(0, cb.numel() - 1), idx.clamp(0, cb.numel() - 1)
        pick = torch.where((ac - cb[lo]).abs() <= (ac - cb[hi]).abs(), lo, hi)
        mse = ((ac - cb[pick]).square() * stats["active_counts"]).sum().item() / total
        print("  exact DP: MSE_normalized={:.6e}".format(mse))
    return codebook


def _preflight_torch_groups(optimizer, saved_groups) -> None:
    """torch.optim.Optimizer.load_state_dict's own refusals, made before any
    load: the number of parameter groups and each group's size."""
    groups = optimizer.param_groups
    if len(groups) != len(saved_groups):
        raise ValueError("loaded state dict has a different number of parameter groups")
    if any(len(g["params"]) != len(sg["params"]) for g, sg in zip(groups, saved_groups)):
        raise ValueError("loaded state dict contains a parameter group that doesn't match the size of "
                         "optimizer's group")


class Gefen(torch.optim.Optimizer):
    """Gefen optimizer (see module docstring).

    Args mirror the reference (gefen.py:1074-1092): ``lr``, ``betas``, ``eps``,
    ``weight_decay``, and keyword-only ``fused``, ``force_1d_period_one``,
    ``force_2d_period_one``, ``period_one_substrings``, ``factored_v_2d``,
    ``codebook_refresh_every``, ``stochastic_round``, ``deterministic``,
    ``capturable``, ``verbose``.
    """

    def __init__(
        self,
        params: Iterable[Union[nn.Parameter, Tuple[str, nn.Parameter]]],
        lr: Union[float, torch.Tensor] = 1e-3,
        betas: Tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 0.0,
        *,
        fused: bool = True,
        force_1d_period_one: bool = False,
        force_2d_period_one: bool = False,
        period_one_substrings: Tuple[str, ...] = (),
        factored_v_2d: bool = True,
        codebook_refresh_every: int = 0,
        stochastic_round: bool = False,
        deterministic: bool = False,
        capturable: bool = False,
        verbose: bool = False,
    ):
        if not isinstance(deterministic, bool):
            raise TypeError("deterministic must be a bool")
        if deterministic and factored_v_2d and stochastic_round:
            raise ValueError(
                "deterministic=True with factored_v_2d=True cannot honor stochastic_round=True: the "
                "replica-exact factored path uses deterministic nearest-codeword quantization. Disable "
                "stochastic rounding or factored_v_2d.")
        self._validate_group_options(lr, betas, eps, weight_decay)
        if codebook_refresh_every < 0:
            raise ValueError("codebook_refresh_every must be >= 0 but is: {}".format(codebook_refresh_every))
        if capturable and codebook_refresh_every:
            raise ValueError("capturable=True is incompatible with codebook_refresh_every>0: the periodic "
                             "codebook re-learn is host-driven and cannot run inside a replayed CUDA graph.")
        # fused=False is the same step here (the decomposed step's arithmetic is
        # what the kernels compute); the flag is kept for the reference's API.
        self.fused = bool(fused)
        self._force_1d_period_one = force_1d_period_one
        self._force_2d_period_one = force_2d_period_one
        self._period_one_substrings = tuple(s.lower() for s in period_one_substrings)
        self._factored_v_2d = factored_v_2d
        self._deterministic = deterministic
        self._codebook_refresh_every = codebook_refresh_every
        self.capturable = capturable
        # device step counters / scalar rows / launch plans (subclasses with
        # their own step may turn this off)
        self._capt_on = capturable
        self._stochastic_round = stochastic_round
        self.verbose = verbose
        self._gefen_codebook = None
        self._gefen_codebook_by_device = {}
        self._lr_scalar_cache = None  # (tensor lr, its _version, its value): see _lr_scalar
        self._gefen_global_step = 0
        self._param_names = {}
        # All parameters of a device go through one gefenx_multi_tensor_step
        # call; GEFENX_MULTI_TENSOR=0 selects one call per parameter.
        self._multi_tensor = os.environ.get("GEFENX_MULTI_TENSOR", "1") != "0"
        self._mt_scratch = {}
        # capturable=True: per device an int64[3] {global step, next rounding
        # seed, seed of the running step} advanced on the device each step,
        # and the launch plans of the tensor sets stepped so far.
        self._capt_counters = {}
        self._gefen_global_step_by_device = {}
        self._sr_seed_by_device = {}
        self._capt_plans = OrderedDict()
        # host-resident parameters (CPU offload): pinned / device staging
        # arenas, and each such parameter's device workspace
        self._host_stager = host_staging.HostStager()
        self._offload_ws = {}  # id(p) -> (weak reference to p, workspace)
        defaults = dict(lr=lr, beta1=betas[0], beta2=betas[1], eps=eps, weight_decay=weight_decay)
        super().__init__(self._normalize_param_groups(params), defaults)

    # ------------------------------------------------------------ groups

    @staticmethod
    def _validate_group_options(lr, betas, eps, weight_decay):
        """gefen.py:1254-1275: the lr (a number or a 1-element tensor), betas
        in [0, 1), weight_decay >= 0, eps finite and > 0."""
        if torch.is_tensor(lr) and lr.numel() != 1:
            raise ValueError("lr as a Tensor must be 1-element, got numel={}".format(lr.numel()))
        lr_val = float(lr.item()) if torch.is_tensor(lr) else lr
        if not 0.0 <= lr_val:
            raise ValueError("Invalid learning rate: {}".format(lr_val))
        if len(betas) != 2:
            raise ValueError("betas must be a pair")
        if not 0.0 <= betas[0] < 1.0:
            raise ValueError("Invalid beta parameter at index 0: {}".format(betas[0]))
        if not 0.0 <= betas[1] < 1.0:
            raise ValueError("Invalid beta parameter at index 1: {}".format(betas[1]))
        if not 0.0 <= weight_decay:
            raise ValueError("Invalid weight_decay value: {}".format(weight_decay))
        if not math.isfinite(eps) or eps <= 0.0:
            raise ValueError("Invalid epsilon value: {}; eps must be finite and > 0".format(eps))

    # A group's unnamed parameters are called <prefix><index>: "param_" in the
    # implicit group of a plain parameter list, "group_<g>_param_" otherwise.
    _PREFIX_KEY = "_gefenx_name_prefix"

    def _normalize_param_groups(self, params):
        """gefen.py:1242-1251: a single tensor, an iterable of tensors or of
        (name, tensor) pairs (one implicit group), or an iterable of group
        dicts.  Each group then goes through add_param_group."""
        if isinstance(params, torch.Tensor):
            params = [params]
        params = list(params)
        if len(params) == 0:
            raise ValueError("optimizer got an empty parameter list")
        if isinstance(params[0], dict):
            return [dict(g, **{self._PREFIX_KEY: "group_{}_param_".format(i)}) for i, g in enumerate(params)]
        return [{"params": params, self._PREFIX_KEY: "param_"}]

    def _split_names(self, items, prefix, group_name=None):
        """(names, tensors, synthesized flags) of a group's params, checked and
        named without registering anything (add_param_group registers the
        names once the whole group is valid).  gefen.py:1451-1499: a given
        name is lowercased and kept as is (two parameters may share one; their
        states stay separate); an unnamed parameter alone in a group with a
        "name" takes that name, otherwise its positional <prefix><index>; a
        generated name that is already taken gets the first free _<n> suffix
        and counts as synthesized."""
        if isinstance(items, torch.Tensor):
            items = [items]
        items = list(items)
        names, ps, synth = [], [], []
        seen = set(self._param_names.values())

        def free(base):
            if base not in seen:
                return base
            k = 1
            while "{}_{}".format(base, k) in seen:
                k += 1
            return "{}_{}".format(base, k)

        for i, it in enumerate(items):
            if isinstance(it, (tuple, list)) and len(it) == 2 and isinstance(it[0], str):
                name, p, generated = str(it[0]).lower(), it[1], False
            elif group_name is not None and len(items) == 1:
                base = str(group_name).lower()
                name, p = free(base), it
                generated = name != base
            else:
                name, p, generated = free("{}{}".format(prefix, i)), it, True
            if not isinstance(p, torch.Tensor):
                raise TypeError("Gefen can only optimize Tensors, but one of the params is {}".format(
                    type(p).__name__))
            if torch.is_complex(p):
                raise ValueError("Gefen does not support complex parameters, but got a parameter with dtype "
                                 "{}".format(p.dtype))
            seen.add(name)
            names.append(name)
            ps.append(p)
            synth.append(generated)
        return names, ps, synth

    def _check_group_params(self, params):
        """Subclass hook: reject parameters this optimizer cannot step."""

    def add_param_group(self, param_group):
        """gefen.py:1388-1525: all or nothing.  Hyperparameters (group value or
        the constructor's), parameter types and duplicates (inside the group
        and against the existing groups) are checked before anything is
        registered; unnamed parameters get positional names."""
        if not isinstance(param_group, dict):
            raise TypeError("param_group must be a dict, got {}".format(type(param_group).__name__))
        if "params" not in param_group:
            raise ValueError("Gefen parameter group is missing the 'params' key.")
        g = dict(param_group)
        prefix = g.pop(self._PREFIX_KEY, "group_{}_param_".format(len(self.param_groups)))
        if "betas" in g:
            g["beta1"], g["beta2"] = g.pop("betas")
        d = self.defaults
        self._validate_group_options(g.get("lr", d["lr"]), (g.get("beta1", d["beta1"]), g.get("beta2", d["beta2"])),
                                     g.get("eps", d["eps"]), g.get("weight_decay", d["weight_decay"]))
        names, ps, synth = self._split_names(g["params"], prefix, g.get("name"))
        if len(ps) == 0:
            raise ValueError("optimizer got an empty parameter list")
        if g.get("name") is not None:
            g["name"] = str(g["name"]).lower()
        elif len(names) == 1:
            g["name"] = names[0]
        self._check_group_params(ps)
        existing = {id(p) for grp in self.param_groups for p in grp["params"]}
        batch = set()
        for p in ps:
            if id(p) in existing or id(p) in batch:
                raise ValueError("some parameters appear in more than one parameter group")
            batch.add(id(p))
        g["params"], g["param_names"], g["param_names_synthesized"] = ps, names, synth
        super().add_param_group(g)
        for p, name in zip(ps, names):
            self._param_names[p] = name
            self.state[p]["name"] = name  # gefen.py:1520-1525: every state carries its parameter's name

    def _iter_group_params_with_names(self, group):
        names = group.get("param_names") or [self._param_names.get(p, "param") for p in group["params"]]
        return zip(names, group["params"])

    # ---------------------------------------------------------- codebook

    def _gefen_codebook_on(self, device):
        cb = self._gefen_codebook
        if cb is None or cb.device == device:
            return cb
        cached = self._gefen_codebook_by_device.get(device)
        if cached is None:
            cached = cb.to(device)
            self._gefen_codebook_by_device[device] = cached
        return cached

    def _resolve_automatic_period(self, param_name, param, grad) -> int:
        """gefen.py:2563-2577 (force flags, then the block-variance search)."""
        if self._force_1d_period_one and param.ndim == 1:
            return 1
        if self._force_2d_period_one and param.ndim == 2:
            return 1
        if self._period_one_substrings:
            lname = str(param_name).lower()
            if any(s in lname for s in self._period_one_substrings):
                return 1
        flat = grad.detach().reshape(-1)
        if flat.numel() == 1:
            return 1
        if flat.device.type == "cpu":  # a host-resident parameter: the search runs on the GPU
            flat = flat.to(self._compute_device())
        return partitioning.find_period_by_block_variance(
            flat, print_results=False, parameter_name=param_name, parameter_shape=tuple(param.shape),
            backend="cuda_kernel", input_is_squared=False)

    def _iter_gefen_grad_periods(self, reuse_existing_periods=False):
        for group in self.param_groups:
            for name, p in self._iter_group_params_with_names(group):
                if p.grad is None:
                    continue
                grad = p.grad.detach()
                flat = grad.reshape(-1)
                if flat.numel() == 0:
                    continue
                state = self.state[p]
                if reuse_existing_periods and "automatic_period" in state:
                    period = state["automatic_period"]
                elif "automatic_period" in state:
                    period = state["automatic_period"]
                elif flat.numel() == 1:
                    period = 1
                else:
                    period = self._resolve_automatic_period(name, p, grad)
                state["automatic_period"] = int(period)
                if flat.numel() % period != 0:
                    raise ValueError("Automatic partition period {} does not divide parameter {} with numel {} "
                                     "while learning Gefen codebook".format(period, name, flat.numel()))
                yield name, flat, int(period), grad

    def _device_grad_periods(self, reuse_existing_periods=False, homes=None):
        """_iter_gefen_grad_periods with every flat gradient on a HIP device:
        a host-resident gradient is copied to the compute device one tensor
        at a time, as the consumer reaches it (the histogram kernel reads it
        there).  `homes`, when given, collects each gradient's own device."""
        for name, flat, period, grad in self._iter_gefen_grad_periods(reuse_existing_periods):
            if homes is not None:
                homes.append(grad.device)
            if flat.device.type == "cpu":
                flat = flat.to(self._compute_device())
            yield name, flat, period, grad

    def _grad_histogram_counts(self, bins, reuse_existing_periods=False):
        """The step-1 histogram over this optimizer's gradients (gefen.py:
        417-469): (int64 counts on the device, number of elements), or
        (None, 0) when no parameter has a gradient."""
        return _exact_histogram_counts(self._device_grad_periods(reuse_existing_periods), bins)

    def _learn_gefen_exact_codebook(self, reuse_existing_periods=False):
        """learn_gefen_exact_codebook_from_grad_periods (gefen.py:417-517)
        over this optimizer's gradients: the 256-entry codebook, endpoints
        forced; None without gradients.  Returns (codebook on the first
        gradient's own device, as the reference keeps it, or None; the same
        values on the device the histogram ran on)."""
        homes = []
        cb = learn_gefen_exact_codebook_from_grad_periods(
            grad_periods=self._device_grad_periods(reuse_existing_periods, homes), codebook_device=None,
            num_codebooks=NUM_CODEBOOKS, force_endpoints=True, verbose=False, compute_mse_logging=False)
        if cb is None:
            return None, None
        return (cb if homes[0] == cb.device else cb.to(homes[0])), cb

    def _adopt_codebook(self, home, computed):
        """Make `home` the codebook; keep the copy on the compute device."""
        self._gefen_codebook = home
        self._gefen_codebook_by_device.clear()
        if computed is not None and computed.device != home.device:
            self._gefen_codebook_by_device[computed.device] = computed

    def _maybe_save_gefen_grad_histogram(self):
        """gefen.py:3095-3150: at the global steps listed in
        quantization.LIST_STEPS_SAVE_HIST_GRAD, write the histogram of the
        block-absmax-normalised gradients (codebook size x 16 bins) next to
        quantization.SAVE_CODEBOOK_PREFIX; the counts come from the histogram
        kernel (its binning equals the reference's for power-of-two bin
        counts, e.g. 4096 for a 256-entry codebook)."""
        steps = getattr(quantization_module, "LIST_STEPS_SAVE_HIST_GRAD", None)
        if steps is None:
            return
        if self.capturable and steps:
            raise ValueError("capturable=True is incompatible with LIST_STEPS_SAVE_HIST_GRAD: histogram collection "
                             "and file output are host-driven")
        if self._gefen_global_step not in steps:
            return
        prefix = getattr(quantization_module, "SAVE_CODEBOOK_PREFIX", None)
        if prefix is None:
            raise ValueError("LIST_STEPS_SAVE_HIST_GRAD requires SAVE_CODEBOOK_PREFIX to be set.")
        if self._gefen_codebook is None:
            raise ValueError("Expected Gefen codebook to be initialized before saving gradient histogram.")
        bins = self._gefen_codebook.numel() * 16
        counts_dev, total = self._grad_histogram_counts(bins, reuse_existing_periods=True)
        if total == 0:
            raise ValueError("Cannot save Gefen gradient histogram because no gradients were available.")
        quantization_module.save_distribution_histogram_pt_from_counts(
            hist=counts_dev.cpu().to(torch.float32), prefix=prefix,
            suffix="grad_hist_step_{}".format(self._gefen_global_step), num_samples=total)

    def _maybe_refresh_gefen_codebook(self):
        if self._gefen_codebook is not None:
            return
        cb, computed = self._learn_gefen_exact_codebook(
            reuse_existing_periods=any("automatic_period" in self.state.get(p, {})
                                       for g in self.param_groups for p in g["params"]))
        if cb is not None:
            self._adopt_codebook(cb, computed)

    def _refresh_codebook_with_requant(self):
        """gefen.py:3020-3070: re-learn, then map stored indices onto the new
        codebook through nearest-codeword search of the old coefficients."""
        old = self._gefen_codebook
        if old is None:
            return
        new, computed = self._learn_gefen_exact_codebook(reuse_existing_periods=True)
        if new is None:
            return
        old_h = old.detach().cpu().float().numpy()
        new_h = new.detach().cpu().float()
        remap = torch.searchsorted(new_h, torch.from_numpy(old_h))
        k = new_h.numel()
        left = (remap - 1).clamp(0, k - 1)
        right = remap.clamp(0, k - 1)
        x = torch.from_numpy(old_h)
        choose = torch.where((x - new_h[left]).abs() <= (x - new_h[right]).abs(), left, right).to(torch.uint8)
        # every remapped index tensor is built before any is written, so a
        # failure part-way leaves the indices and the codebook as they were
        staged = []
        for group in self.param_groups:
            for p in group["params"]:
                st = self.state.get(p)
                if st and "m_codebook" in st:
                    staged.append((st["m_codebook"], choose.to(st["m_codebook"].device)[st["m_codebook"].long()]))
        for dst, src in staged:
            dst.copy_(src)
        self._adopt_codebook(new, computed)

    # -------------------------------------------------------------- step

    def _validate_grads(self):
        """gefen.py:897-981: reject bad grads before mutating anything."""
        for group in self.param_groups:
            for name, p in self._iter_group_params_with_names(group):
                g = p.grad
                if g is None:
                    continue
                if getattr(g, "is_sparse", False) or g.layout != torch.strided:
                    raise RuntimeError("Gefen does not support sparse gradients")
                if torch.is_complex(g):
                    raise RuntimeError("Gefen does not support complex gradients")
                if g.shape != p.shape:
                    raise RuntimeError("gradient shape {} does not match parameter {} shape {}".format(
                        tuple(g.shape), name, tuple(p.shape)))
                if g.device != p.device:
                    raise RuntimeError("gradient and parameter {} must be on the same device: gradient on {}, "
                                       "parameter on {}".format(name, g.device, p.device))
                if p.numel() and p.device.type != "cuda":
                    self._check_host_parameter(name, p)
                if p.dtype == torch.float64:
                    raise NotImplementedError("Gefen fused kernels are not implemented for 'Double' ({})".format(name))
                if g.dtype != p.dtype:
                    raise RuntimeError("gradient dtype {} does not match parameter {} dtype {}".format(
                        g.dtype, name, p.dtype))

    # Whether parameters in host memory are stepped (through the pinned
    # staging of gefen/host_staging.py); subclasses whose step has no staged
    # path turn it off.
    _steps_host_params = True

    def _check_host_parameter(self, name, p):
        """A parameter that is not on a HIP device: host memory is stepped on
        the compute device through pinned staging (CPU offload, reference
        gefen.py:1897-1927); anything else, or host memory without a HIP
        device, or under capturable (a graph cannot record host memory), is
        refused before anything mutates."""
        if p.device.type != "cpu" or not self._steps_host_params:
            raise RuntimeError("Gefen (MI355X build) steps HIP device parameters only; {} is on {}".format(
                name, p.device))
        if self.capturable:
            raise RuntimeError("Gefen capturable=True steps HIP device parameters only; {} is in host memory "
                               "(CUDA-graph capture cannot record host-resident tensors)".format(name))
        if not torch.cuda.is_available():
            raise RuntimeError("Gefen (MI355X build) steps host-resident parameters on a HIP device, and none is "
                               "available ({} is on {})".format(name, p.device))

    @staticmethod
    def _compute_device():
        """The HIP device that steps host-resident parameters: the current one."""
        return torch.device("cuda", torch.cuda.current_device())

    def _lr_scalar(self, group) -> float:
        """group["lr"] as a python float (gefen.py:1530-1555).  A tensor lr is
        read from the device only when it is a different tensor or its
        _version moved (an in-place scheduler update) since the last read:
        one slot for all groups, so a constant or once-per-step-updated device
        lr costs at most one host sync per step, not one per parameter, and a
        fresh tensor per step cannot grow the cache.  Kept out of param_groups
        and the state_dict."""
        lr = group["lr"]
        if not torch.is_tensor(lr):
            return float(lr)
        hit = getattr(self, "_lr_scalar_cache", None)
        if hit is not None and hit[0] is lr and hit[1] == lr._version:
            return hit[2]
        value = float(lr.item())
        self._lr_scalar_cache = (lr, lr._version, value)
        return value

    def _init_state(self, state, p, grad, name, factored):
        numel = grad.numel()
        if "automatic_period" in state:
            period = int(state["automatic_period"])
        elif numel == 1:
            period = 1
        else:
            period = self._resolve_automatic_period(name, p, grad)
        if numel % period != 0:
            raise ValueError("Automatic partition period {} does not divide parameter {} with numel {}".format(
                period, name, numel))
        nb = numel // period
        state["automatic_period"] = period
        state["step"] = self._new_step_counter(p.device)
        state["m_codebook"] = torch.zeros(nb, period, dtype=torch.uint8, device=p.device)
        state["m_magnitude"] = torch.zeros(nb, 1, dtype=torch.float32, device=p.device)
        if factored:
            state["v_row"] = torch.zeros(p.shape[0], dtype=torch.float32, device=p.device)
            state["v_col"] = torch.zeros(p.shape[1], dtype=torch.float32, device=p.device)
            state["factored_step"] = self._new_step_counter(p.device)
        else:
            state["vmean"] = torch.zeros(nb, 1, dtype=torch.float32, device=p.device)
            state["vmean_step"] = self._new_step_counter(p.device)

    def _colocate_param_state_(self, state, device: torch.device) -> None:
        """gefen.py:1897-1927: a parameter relocated between steps (CPU offload
        paging it CPU -> GPU, or a move to another GPU) finds its state on the
        previous device; move the state tensors to the parameter's device.
        Same-device steps return after one device compare (no copy, no
        reassignment).  Under capturable the state addresses are part of the
        recorded launches, so nothing moves."""
        if self.capturable:
            return
        sentinel = state.get("m_codebook")
        if sentinel is None or sentinel.device == device:
            return
        for key in _COLOCATABLE_STATE_KEYS:
            value = state.get(key)
            if torch.is_tensor(value) and value.device != device:
                state[key] = value.to(device)  # a pure copy: indices and magnitudes move bit for bit

    def _new_step_counter(self, device, value=0):
        """gefen.py:1887-1895: a python int, or under capturable a 0-dim fp32
        device tensor so the bias corrections are computed on the device."""
        if self._capt_on:
            return torch.full((), float(value), dtype=torch.float32, device=device)
        return int(value)

    def _workspace(self, state, kind, rows, cols, nb, device):
        ws = state.get("_gefenx_ws")
        need = int(_native.load().gefenx_workspace_bytes(kind, rows, cols, nb))
        if ws is None or ws.numel() < need or ws.device != device:
            ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)
            state["_gefenx_ws"] = ws
        return ws

    def _prepare_factored(self, group, name, p, grad):
        """State bookkeeping of gefen.py:2784-2852 (lazy init, resume from a
        block-vmean checkpoint, step counters); returns the kernel scalars."""
        state = self.state[p]
        if "step" not in state:
            self._init_state(state, p, grad, name, factored=True)
        self._colocate_param_state_(state, grad.device)
        if "v_row" not in state:  # resume from a block-vmean checkpoint (gefen.py:2840-2852)
            state["v_row"] = torch.zeros(p.shape[0], dtype=torch.float32, device=p.device)
            state["v_col"] = torch.zeros(p.shape[1], dtype=torch.float32, device=p.device)
            state["factored_step"] = self._new_step_counter(p.device)
        if self._capt_on:  # counters and scalars advance on the device
            return state, None, None, None, None, 0.0
        state["step"] += 1
        state["factored_step"] += 1
        lr = self._lr_scalar(group)
        bc1 = 1 - group["beta1"] ** state["step"]
        bc2 = 1 - group["beta2"] ** state["factored_step"]
        # and the divisor bc2, as the kernels' C entry points derive it from
        # 1/bc2 (the kernels divide by it, as the reference's step does)
        inv_bc2 = 1.0 / bc2
        return state, lr, inv_bc2, 1.0 / bc1, 1.0 - lr * group["weight_decay"], 1.0 / inv_bc2

    def _prepare_block(self, group, name, p, grad):
        """State bookkeeping of gefen.py:3488-3586; returns the kernel scalars
        (the second one is 1/sqrt(bc2), as the block stepsize uses it)."""
        state = self.state[p]
        if "step" not in state:
            self._init_state(state, p, grad, name, factored=False)
        self._colocate_param_state_(state, grad.device)
        if "vmean" not in state:  # resume from a factored checkpoint (gefen.py:3567-3586)
            state["vmean"] = torch.zeros_like(state["m_magnitude"])
            state["vmean_step"] = self._new_step_counter(p.device)
        elif "vmean_step" not in state:
            step = state["step"]
            state["vmean_step"] = step.clone() if torch.is_tensor(step) else step
        if self._capt_on:
            return state, None, None, None, None, 0.0
        state["step"] += 1
        state["vmean_step"] += 1
        lr = self._lr_scalar(group)
        bc1 = 1 - group["beta1"] ** state["step"]
        bc2 = 1 - group["beta2"] ** state["vmean_step"]
        inv_sqrt_bc2 = 1.0 / math.sqrt(bc2)
        return state, lr, inv_sqrt_bc2, 1.0 / bc1, 1.0 - lr * group["weight_decay"], 1.0 / inv_sqrt_bc2

    def _step_automatic_factored(self, group, name, p, grad, prepared=None):
        """gefen.py:2784-3018 on the MI355X factored kernels (one parameter)."""
        if grad.numel() == 0:
            return
        state, lr, inv_bc2, inv_bc1, wdf, _ = prepared or self._prepare_factored(group, name, p, grad)
        scalars_ptr, seed_ptr = self._capt_pointers(state, p.device)
        if scalars_ptr is not None:
            lr, inv_bc2, inv_bc1, wdf = 0.0, 1.0, 1.0, 1.0
        rows, cols = p.shape
        period = state["automatic_period"]
        nb = p.numel() // period
        ws = self._workspace(state, _native.WS_FACTORED, rows, cols, nb, p.device)
        qt = _fused.quant_table(self._gefen_codebook_on(p.device), p.dtype)
        _native.check(_native.load().gefenx_factored_update(
            p.data_ptr(), grad.data_ptr(), _fused._dtype_code(p.dtype), rows, cols,
            p.stride(0), p.stride(1), grad.stride(0), grad.stride(1),
            state["m_codebook"].data_ptr(), state["m_magnitude"].data_ptr(),
            state["v_row"].data_ptr(), state["v_col"].data_ptr(), period, qt.data_ptr(),
            group["beta1"], group["beta2"], lr, group["eps"], inv_bc2, inv_bc1, wdf,
            1 if self._stochastic_round else 0, self._kernel_rng_seed(), scalars_ptr, seed_ptr,
            ws.data_ptr(), ws.numel(), _stream_of(p)), "factored update of " + name)

    def _step_automatic(self, group, name, p, grad, prepared=None):
        """gefen.py:3488-3818 on the MI355X block kernels (one parameter)."""
        if grad.numel() == 0:
            return
        state, lr, inv_sqrt_bc2, inv_bc1, wdf, _ = prepared or self._prepare_block(group, name, p, grad)
        scalars_ptr, seed_ptr = self._capt_pointers(state, p.device)
        if scalars_ptr is not None:
            lr, inv_sqrt_bc2, inv_bc1, wdf = 0.0, 1.0, 1.0, 1.0
        period = state["automatic_period"]
        nb = p.numel() // period
        p_k = p if p.is_contiguous() else p.contiguous()
        g_k = grad if grad.is_contiguous() else grad.contiguous()
        ws = self._workspace(state, _native.WS_BLOCK, 1, p.numel(), nb, p.device)
        qt = _fused.quant_table(self._gefen_codebook_on(p.device), p.dtype)
        _native.check(_native.load().gefenx_block_update(
            p_k.data_ptr(), g_k.data_ptr(), _fused._dtype_code(p.dtype), p.numel(), period,
            state["m_codebook"].data_ptr(), state["m_magnitude"].data_ptr(), state["vmean"].data_ptr(),
            qt.data_ptr(), group["beta1"], group["beta2"], lr, group["eps"], inv_sqrt_bc2, inv_bc1, wdf,
            1 if self._stochastic_round else 0, self._kernel_rng_seed(), scalars_ptr, seed_ptr,
            ws.data_ptr(), ws.numel(), _stream_of(p)), "block update of " + name)
        if p_k is not p:
            p.copy_(p_k)

    def _desc_row(self, group, p, grad, factored, prepared):
        """One gefenx_tensor_desc (include/gefenx.h) as a tuple in field order."""
        state = prepared[0]
        nb = p.numel() // state["automatic_period"]
        if factored:
            rows, cols = p.shape
            ws = self._workspace(state, _native.WS_FACTORED, rows, cols, nb, p.device)
            v0, v1 = state["v_row"].data_ptr(), state["v_col"].data_ptr()
            strides = (p.stride(0), p.stride(1), grad.stride(0), grad.stride(1))
        else:
            ws = self._workspace(state, _native.WS_BLOCK, 1, p.numel(), nb, p.device)
            v0, v1 = state["vmean"].data_ptr(), 0
            if p.is_contiguous() and grad.is_contiguous():
                rows, cols = 1, p.numel()
                strides = (cols, 1, cols, 1)
            else:  # a transposed view (_block_view_ok): logical [rows, cols]
                rows, cols = p.shape
                strides = (p.stride(0), p.stride(1), grad.stride(0), grad.stride(1))
        return self._desc_fields(group, prepared, factored, p.dtype, rows, cols, strides, p.data_ptr(),
                                 grad.data_ptr(), state["m_codebook"].data_ptr(),
                                 state["m_magnitude"].data_ptr(), v0, v1, ws.data_ptr())

    @staticmethod
    def _desc_fields(group, prepared, factored, dtype, rows, cols, strides, p_ptr, g_ptr, idx_ptr, mag_ptr,
                     v0, v1, ws_ptr):
        state, lr, inv_bc2, inv_bc1, wdf, bc2_div = prepared
        if lr is None:  # capturable: the tensor reads its scalar row on the device
            lr, inv_bc2, inv_bc1, wdf, bc2_div = 0.0, 1.0, 1.0, 1.0, 0.0
        beta1, beta2 = group["beta1"], group["beta2"]
        return (p_ptr, g_ptr, idx_ptr, mag_ptr, v0, v1, ws_ptr, rows, cols) + tuple(strides) + (
            state["automatic_period"], _fused._dtype_code(dtype), 1 if factored else 0,
            lr, group["eps"], inv_bc2, inv_bc1, wdf, 1.0 - beta1, beta2, 1.0 - beta2, bc2_div)

    def _launch_staged(self, device, items, arena):
        """One multi-tensor launch over a chunk of host-resident parameters
        whose parameter, gradient and state copies sit in `arena` (device
        bytes laid out by host_staging); their workspaces stay on the device
        between steps, outside the state dict (the state follows the
        parameter to the host)."""
        base = arena.data_ptr()
        rows, dtypes = [], set()
        for it in items:
            state, p = it.prepared[0], it.p
            at = {key: base + off for key, _, off in it.pieces}
            nb = p.numel() // state["automatic_period"]
            if it.factored:
                r, c = p.shape
                kind, wr, wc = _native.WS_FACTORED, r, c
                v0, v1 = at["v_row"], at["v_col"]
            else:
                r, c = 1, p.numel()
                kind, wr, wc = _native.WS_BLOCK, 1, c
                v0, v1 = at["vmean"], 0
            need = int(_native.load().gefenx_workspace_bytes(kind, wr, wc, nb))
            ref, ws = self._offload_ws.get(id(p), (None, None))
            if ref is None or ref() is not p or ws.numel() < need or ws.device != device:
                for key in [k for k, (r, _) in self._offload_ws.items() if r() is None]:
                    del self._offload_ws[key]  # parameters that no longer exist
                ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)
                self._offload_ws[id(p)] = (weakref.ref(p), ws)
            rows.append(self._desc_fields(it.group, it.prepared, it.factored, p.dtype, r, c, (c, 1, c, 1),
                                          at["p"], base + it.grad_offset, at["m_codebook"], at["m_magnitude"],
                                          v0, v1, ws.data_ptr()))
            dtypes.add(p.dtype)
        self._multi_tensor_step(device, rows, dtypes)

    def _multi_tensor_step(self, device, rows, dtypes):
        """All parameters of one device in one gefenx_multi_tensor_step call
        (stats, finalize and apply phases each launched once per kernel
        variant instead of once per parameter)."""
        lib = _native.load()
        descs = np.array(rows, dtype=_DESC_DTYPE)
        cb = self._gefen_codebook_on(device)
        qt = [0, 0, 0]
        for dt in dtypes:
            qt[_fused._dtype_code(dt)] = _fused.quant_table(cb, dt).data_ptr()
        qt_arr = (ctypes.c_void_p * 3)(*qt)
        need = int(lib.gefenx_multi_tensor_scratch_bytes(len(rows)))
        scratch = self._mt_scratch.get(device)
        if scratch is None or scratch.numel() < need:
            scratch = torch.empty(need, dtype=torch.uint8, device=device)
            self._mt_scratch[device] = scratch
        with torch.cuda.device(device):
            _native.check(lib.gefenx_multi_tensor_step(
                descs.ctypes.data, len(rows), qt_arr, 1 if self._stochastic_round else 0,
                self._gefen_global_step, scratch.data_ptr(), scratch.numel(),
                torch.cuda.current_stream(device).cuda_stream), "multi-tensor step")

    # -------------------------------------------------------- capturable

    def _kernel_rng_seed(self) -> int:
        """gefen.py:1755-1768: the host rounding seed; under capturable the
        kernels read it from the device counter instead."""
        return 0 if self._capt_on else self._gefen_global_step

    @property
    def _step_supports_amp_scaling(self) -> bool:
        """gefen.py:1233-1239: GradScaler asks this before its overflow scan;
        true fp16 gradients take the native protocol handled in ``step``."""
        return _amp_native_scaling_required(self)

    def _assert_capturable_if_capturing(self) -> bool:
        """gefen.py:1614-1641; returns whether the current stream is capturing."""
        capturing = torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
        if capturing and not self.capturable:
            raise RuntimeError(
                "Attempting CUDA graph capture of {}.step() but capturable=False. Construct the optimizer "
                "with capturable=True to make step() graph-safe.".format(type(self).__name__))
        if capturing:
            devices = {p.device for g in self.param_groups for p in g["params"]}
            capture_device = torch.device("cuda", torch.cuda.current_device())
            if devices != {capture_device}:
                raise RuntimeError("CUDA graph capture requires every Gefen parameter on the current capture "
                                   "device {}; found {}".format(capture_device, sorted(map(str, devices))))
        return capturing

    def _cuda_param_devices(self):
        return sorted({p.device for g in self.param_groups for p in g["params"] if p.device.type == "cuda"},
                      key=lambda d: -1 if d.index is None else d.index)

    def _ensure_gefen_global_step_devices(self):
        """gefen.py:1826-1853: one device counter per parameter device, created
        eagerly (a counter created inside a capture would be reset by every
        replay)."""
        if not self._capt_on:
            return
        for device in self._cuda_param_devices():
            if device in self._capt_counters:
                continue
            buf = torch.full((3,), int(self._gefen_global_step), dtype=torch.int64, device=device)
            self._capt_counters[device] = buf
            self._gefen_global_step_by_device[device] = buf[0]
            if self._stochastic_round:
                self._sr_seed_by_device[device] = buf[1]

    def _reset_gefen_global_step_devices(self):
        self._capt_counters.clear()
        self._gefen_global_step_by_device.clear()
        self._sr_seed_by_device.clear()
        self._capt_plans_clear()
        self._ensure_gefen_global_step_devices()

    def _device_gefen_global_step(self):
        steps = [int(buf[0].item()) for buf in self._capt_counters.values()]
        if any(s != steps[0] for s in steps[1:]):
            raise RuntimeError("Gefen capturable global-step counters disagree across devices: {}".format(steps))
        return steps[0] if steps else None

    def _synchronize_gefen_global_step_for_checkpoint(self):
        """gefen.py:1855-1870: the host mirror from the device counter after
        graph replays."""
        if not self._capt_on:
            return
        self._ensure_gefen_global_step_devices()
        device_step = self._device_gefen_global_step()
        if device_step is not None:
            self._gefen_global_step = device_step

    def _assert_capture_ready(self):
        if self._gefen_codebook is None and any(p.grad is not None and p.numel()
                                                for g in self.param_groups for p in g["params"]):
            raise RuntimeError("{} capturable: step 1 (period search and codebook learning) runs on the host; "
                               "run at least one eager step() before capturing".format(type(self).__name__))
        if set(self._cuda_param_devices()) - set(self._capt_counters):
            raise RuntimeError("{} capturable: run one eager step() before capturing (the device step counters "
                               "are created eagerly)".format(type(self).__name__))

    def _capt_pointers(self, state, device):
        """(scalar row pointer, seed pointer) of one tensor under capturable,
        (None, None) otherwise."""
        if not self._capt_on:
            return None, None
        counter = self._capt_counters[device]
        return state["_capt_scalars"].data_ptr(), counter.data_ptr() + 2 * counter.element_size()

    def _capt_ready_state(self, state, p, capturing):
        """Counters as 0-dim fp32 device tensors and the scalar row; inside a
        capture they must already exist (step 1 and state creation run eagerly)."""
        ok = all(torch.is_tensor(state.get(k)) and state[k].device == p.device and state[k].dtype == torch.float32
                 for k in _COUNTER_KEYS if k in state)
        if capturing:
            if not ok or "_capt_scalars" not in state:
                raise RuntimeError("Gefen capturable: a parameter's state was created or converted inside a "
                                   "graph capture; run one eager step() after construction, load_state_dict or "
                                   "a new parameter getting gradients, then capture")
            return
        for k in _COUNTER_KEYS:
            if k in state and not (torch.is_tensor(state[k]) and state[k].device == p.device
                                   and state[k].dtype == torch.float32):
                v = state[k].item() if torch.is_tensor(state[k]) else state[k]
                state[k] = self._new_step_counter(p.device, v)
        if "_capt_scalars" not in state or state["_capt_scalars"].device != p.device:
            state["_capt_scalars"] = torch.ones(4, dtype=torch.float32, device=p.device)

    def _capt_row(self, group, p, state, bc2_key, sqrt_bc2):
        """One gefenx_capt_desc (include/gefenx.h) in field order; bc2_key
        names the counter of the second-moment bias correction (or None)."""
        lr = group["lr"]
        lr_dev, lr_val, lr_code = 0, 0.0, 0
        if torch.is_tensor(lr) and lr.device.type == "cuda":
            if lr.device != p.device:
                raise RuntimeError("capturable tensor lr on {} but parameter on {}".format(lr.device, p.device))
            if lr.dtype not in _LR_DTYPE_CODES:
                raise TypeError("capturable tensor lr of dtype {} (fp32/fp16/bf16/fp64 only)".format(lr.dtype))
            lr_dev, lr_code = lr.data_ptr(), _LR_DTYPE_CODES[lr.dtype]
        else:
            lr_val = float(lr)  # a host value: baked into a captured graph, as for torch.optim
        return (state["step"].data_ptr(), state[bc2_key].data_ptr() if bc2_key else 0,
                state["_capt_scalars"].data_ptr(), lr_dev, lr_val, float(group["weight_decay"]),
                float(group["beta1"]), float(group["beta2"]), lr_code, 1 if sqrt_bc2 else 0)

    def _capt_plans_clear(self):
        plans, self._capt_plans = self._capt_plans, OrderedDict()
        lib = _native.load() if plans else None
        for ent in plans.values():
            if not ent[2]:  # a plan some graph recorded stays alive (its graph may replay)
                lib.gefenx_mt_plan_destroy(ent[0])

    def _capt_launch(self, device, rows, scalar_ptrs, capt_rows, dtypes, capturing):
        """Prologue + multi-tensor phases for one device through a cached plan
        (gefenx_mt_plan_*): kernels only, so the launch can be captured."""
        lib = _native.load()
        counter = self._capt_counters[device]
        cb = self._gefen_codebook_on(device)
        qt = [0, 0, 0]
        tables = []  # the plan bakes these addresses in: it keeps the tensors alive
        for dt in dtypes:
            t = _fused.quant_table(cb, dt)
            tables.append(t)
            qt[_fused._dtype_code(dt)] = t.data_ptr()
        sr = 1 if self._stochastic_round else 0
        key = (device, tuple(rows), tuple(scalar_ptrs), tuple(capt_rows), tuple(qt), sr, counter.data_ptr())
        ent = self._capt_plans.get(key)
        if ent is None:
            n, m = len(rows), len(capt_rows)
            descs = np.array(rows, dtype=_DESC_DTYPE) if n else None
            ss = (ctypes.c_void_p * max(n, 1))(*scalar_ptrs)
            capt = (_native.CaptDesc * max(m, 1))(*[_native.CaptDesc(*r) for r in capt_rows])
            qt_arr = (ctypes.c_void_p * 3)(*qt)
            handle = ctypes.c_void_p()
            with torch.cuda.device(device):
                _native.check(lib.gefenx_mt_plan_create(
                    descs.ctypes.data if n else None, n, ss, qt_arr, sr, 0, capt, m, counter.data_ptr(),
                    ctypes.byref(handle)), "capturable plan")
            nbytes = int(lib.gefenx_mt_plan_device_bytes(handle))
            ent = [handle, torch.empty(nbytes, dtype=torch.uint8, device=device), False, tables]
            self._capt_plans[key] = ent
            if not capturing:
                eager = [k for k, e in self._capt_plans.items() if not e[2] and k != key]
                for k in eager[:max(0, len(eager) - _CAPT_PLAN_CACHE + 1)]:
                    lib.gefenx_mt_plan_destroy(self._capt_plans.pop(k)[0])
        else:
            self._capt_plans.move_to_end(key)
        if capturing:
            ent[2] = True
        with torch.cuda.device(device):
            _native.check(lib.gefenx_mt_plan_launch(ent[0], ent[1].data_ptr(), ent[1].numel(),
                                                    torch.cuda.current_stream(device).cuda_stream),
                          "capturable step")

    # -------------------------------------------------------------- step

    @torch.no_grad()
    def step(self, closure=None):
        capturing = self._assert_capturable_if_capturing()
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        self._validate_grads()
        # gefen.py:5730-5737: a GradScaler overflow returns before the codebook,
        # the state, the counters or the parameters move.
        if not _amp_gate(self):
            return loss
        if capturing:
            self._assert_capture_ready()
        else:
            self._maybe_refresh_gefen_codebook()
            self._maybe_save_gefen_grad_histogram()
            if (self._codebook_refresh_every and self._gefen_global_step > 0
                    and self._gefen_global_step % self._codebook_refresh_every == 0):
                self._refresh_codebook_with_requant()
            self._ensure_gefen_global_step_devices()
        batches = {}  # device -> (desc rows, dtypes, scalar-row pointers, capturable rows)
        deferred = []  # single-tensor launches that read the prologue's scalar rows
        host_items = []  # host-resident parameters (CPU offload)
        for group in self.param_groups:
            for name, p in self._iter_group_params_with_names(group):
                grad = p.grad
                if grad is None or grad.numel() == 0:
                    continue
                factored = self._factored_v_2d and p.ndim == 2 and not hasattr(p, "placements")
                if capturing and "step" not in self.state[p]:
                    raise RuntimeError("Gefen capturable: parameter {} has no state yet; its first step runs "
                                       "eagerly".format(name))
                if factored:
                    prepared = self._prepare_factored(group, name, p, grad)
                else:
                    prepared = self._prepare_block(group, name, p, grad)
                state = prepared[0]
                if p.device.type == "cpu":  # host-resident: stepped below through pinned staging
                    state.pop("_gefenx_ws", None)  # a device workspace does not follow it to the host
                    host_items.append(host_staging.StagedItem(group, name, p, grad, factored, prepared))
                    continue
                # deterministic=True (gefen.py:1048-1057): block-path views
                # take the contiguous route, whose sums run in a fixed order
                # (the view tiles accumulate with atomics)
                batchable = self._multi_tensor and (
                    factored or (p.is_contiguous() and grad.is_contiguous())
                    or (not self._deterministic and _block_view_ok(p, grad, state["automatic_period"])))
                if self._capt_on:
                    self._capt_ready_state(state, p, capturing)
                    rows, dtypes, sptrs, crows = batches.setdefault(p.device, ([], set(), [], []))
                    crows.append(self._capt_row(group, p, state, "factored_step" if factored else "vmean_step",
                                                not factored))
                    if batchable:
                        rows.append(self._desc_row(group, p, grad, factored, prepared))
                        sptrs.append(state["_capt_scalars"].data_ptr())
                        dtypes.add(p.dtype)
                    else:
                        deferred.append((group, name, p, grad, factored, prepared))
                    continue
                if batchable:
                    rows, dtypes, _, _ = batches.setdefault(p.device, ([], set(), [], []))
                    rows.append(self._desc_row(group, p, grad, factored, prepared))
                    dtypes.add(p.dtype)
                elif factored:
                    self._step_automatic_factored(group, name, p, grad, prepared)
                else:
                    self._step_automatic(group, name, p, grad, prepared)
        if self._capt_on:
            for device in self._capt_counters:
                rows, dtypes, sptrs, crows = batches.get(device, ([], set(), [], []))
                self._capt_launch(device, rows, sptrs, crows, dtypes, capturing)
            for group, name, p, grad, factored, prepared in deferred:
                if factored:
                    self._step_automatic_factored(group, name, p, grad, prepared)
                else:
                    self._step_automatic(group, name, p, grad, prepared)
        else:
            for device, (rows, dtypes, _, _) in batches.items():
                self._multi_tensor_step(device, rows, dtypes)
        if host_items:
            device = self._compute_device()
            self._host_stager.run(host_items, device,
                                  lambda items, arena: self._launch_staged(device, items, arena),
                                  host_staging.chunk_bytes_from_env())
        self._gefen_global_step += 1
        return loss

    # -------------------------------------------------------- checkpoint

    def state_dict(self):
        """gefen.py:4558-4707: runtime workspaces stripped; codebook, global
        step and deterministic flag recorded; metadata mirrored per group."""
        self._synchronize_gefen_global_step_for_checkpoint()
        sd = super().state_dict()
        state = {}
        for pid, st in sd["state"].items():
            state[pid] = {k: v for k, v in st.items() if k not in _RUNTIME_STATE_KEYS}
        # every parameter carries its stable name (gefen.py:4562-4565), also
        # before its first step
        for g_saved, g_live in zip(sd["param_groups"], self.param_groups):
            for pid, (name, _) in zip(g_saved["params"], self._iter_group_params_with_names(g_live)):
                entry = state.setdefault(pid, {})
                entry["name"] = entry.get("name", name)
        sd["state"] = {pid: state[pid] for pid in sorted(state)}
        codebook = None if self._gefen_codebook is None else self._gefen_codebook.detach().cpu().clone()
        sd["gefen_global_step"] = self._gefen_global_step
        sd["gefen_deterministic"] = self._deterministic
        sd["gefen_codebook"] = codebook
        anchor = next((p.device for g in self.param_groups for p in g["params"]), torch.device("cpu"))
        meta = {"format_version": _CHECKPOINT_FORMAT_VERSION, "global_step": self._gefen_global_step,
                "codebook": codebook, "deterministic": self._deterministic,
                "device_anchor": torch.zeros(1, dtype=torch.uint8, device=anchor)}
        for g in sd["param_groups"]:
            g["_gefen_checkpoint_metadata"] = meta
        return sd

    def _checkpoint_metadata(self, metas, n_groups, global_step, codebook, deterministic, has_det):
        """Checks of gefen.py:5478-5603: per-group metadata present on all
        groups or none, consistent, agreeing with the top-level keys; the
        replica-determinism policy must match this optimizer's."""
        def same_cb(a, b):
            return a is b or (torch.is_tensor(a) and torch.is_tensor(b) and torch.equal(a.cpu(), b.cpu()))

        if has_det and type(deterministic) is not bool:
            raise ValueError("Gefen checkpoint top-level deterministic policy must be a bool, got {!r}".format(
                deterministic))
        if metas:
            if len(metas) != n_groups:
                raise ValueError("Gefen checkpoint metadata is present on only some parameter groups")
            first = metas[0]
            if first.get("format_version") not in (1, 2):
                raise ValueError("Unsupported Gefen checkpoint metadata format_version: {}".format(
                    first.get("format_version")))
            for m in metas:
                if "deterministic" in m and type(m["deterministic"]) is not bool:
                    raise ValueError("Gefen checkpoint parameter-group deterministic policy must be a bool, "
                                     "got {!r}".format(m["deterministic"]))
            for m in metas[1:]:
                if (m.get("global_step") != first.get("global_step")
                        or not same_cb(m.get("codebook"), first.get("codebook"))
                        or m.get("deterministic") != first.get("deterministic")):
                    raise ValueError("Gefen checkpoint parameter groups carry inconsistent optimizer metadata")
            if global_step is None:
                global_step = first.get("global_step", 0)
            elif global_step != first.get("global_step", 0):
                raise ValueError("Gefen checkpoint top-level and parameter-group global steps disagree")
            if codebook is None:
                codebook = first.get("codebook")
            elif first.get("codebook") is not None and not same_cb(codebook, first.get("codebook")):
                raise ValueError("Gefen checkpoint top-level and parameter-group codebooks disagree")
            if deterministic is None:
                deterministic = first.get("deterministic")
            elif first.get("deterministic") is not None and deterministic != first.get("deterministic"):
                raise ValueError("Gefen checkpoint top-level and parameter-group deterministic policies disagree")
        if deterministic is not None and deterministic != self._deterministic:
            raise ValueError("Gefen checkpoint deterministic={!r}, but this optimizer was constructed with "
                             "deterministic={!r}.  Resuming under another replica-determinism policy requires "
                             "an intentional state migration or a fresh optimizer; refusing to change the "
                             "policy silently.".format(deterministic, self._deterministic))
        return (0 if global_step is None else global_step), codebook, deterministic

    def _preflight_state_dict(self, state_dict) -> None:
        """Every refusal load_state_dict can make, made without changing
        anything: the checkpoint metadata and codebook checks, then torch's
        own group-count and group-size checks.  A composite owner (the hybrid)
        runs this on both halves before loading either (hybrid.py:795-920)."""
        sd = dict(state_dict)
        global_step = sd.pop("gefen_global_step", None)
        has_det = "gefen_deterministic" in sd
        deterministic = sd.pop("gefen_deterministic", None)
        codebook = sd.pop("gefen_codebook", None)
        groups = list(sd.get("param_groups") or [])
        metas = [g["_gefen_checkpoint_metadata"] for g in groups if "_gefen_checkpoint_metadata" in g]
        _, codebook, _ = self._checkpoint_metadata(metas, len(groups), global_step, codebook, deterministic, has_det)
        if any(isinstance(st, dict) and "m_codebook" in st for st in (sd.get("state") or {}).values()) \
                and codebook is None:
            raise ValueError("Gefen checkpoint contains quantized momentum indices but no frozen codebook; loading "
                             "it would reinterpret the restored indices with a different codebook")
        _preflight_torch_groups(self, groups)

    def load_state_dict(self, state_dict):
        """gefen.py:5456-5707: restore saved state dtypes (torch casts floating
        state to the param dtype) and the optimizer-level codebook/step.  The
        load post-hooks run once the whole state (dtypes, names, codebook,
        global step) is in place, not inside torch's part of the load."""
        hooks = self._optimizer_load_state_dict_post_hooks
        self._optimizer_load_state_dict_post_hooks = OrderedDict()
        try:
            self._load_state_dict_raw(state_dict)
        finally:
            self._optimizer_load_state_dict_post_hooks = hooks
        for hook in list(hooks.values()):
            hook(self)

    def _load_state_dict_raw(self, state_dict):
        sd = dict(state_dict)
        global_step = sd.pop("gefen_global_step", None)
        has_det = "gefen_deterministic" in sd
        deterministic = sd.pop("gefen_deterministic", None)
        codebook = sd.pop("gefen_codebook", None)
        metas = []
        groups = []
        for g in sd["param_groups"]:
            g = dict(g)
            m = g.pop("_gefen_checkpoint_metadata", None)
            if m is not None:
                metas.append(m)
            groups.append(g)
        sd["param_groups"] = groups
        global_step, codebook, deterministic = self._checkpoint_metadata(
            metas, len(groups), global_step, codebook, deterministic, has_det)
        if any(isinstance(st, dict) and "m_codebook" in st for st in (sd.get("state") or {}).values()) \
                and codebook is None:
            raise ValueError("Gefen checkpoint contains quantized momentum indices but no frozen codebook; loading "
                             "it would reinterpret the restored indices with a different codebook")
        # torch's loader rebuilds every iterable it meets (a str becomes the
        # text of a generator), so names bypass it
        names = {}
        state = {}
        for pid, st in (sd.get("state") or {}).items():
            st = dict(st)
            if isinstance(st.get("name"), str):
                names[pid] = st.pop("name")
            state[pid] = st
        sd["state"] = state
        saved = {k: {kk: vv for kk, vv in v.items() if torch.is_tensor(vv)} for k, v in sd["state"].items()}
        super().load_state_dict(sd)
        id_map = {}
        for gi, g in enumerate(self.param_groups):
            for p in g["params"]:
                id_map[len(id_map)] = p
        for pid, name in names.items():
            if pid in id_map:
                self.state[id_map[pid]]["name"] = name
        for p in id_map.values():  # a checkpoint without names keeps the registered ones
            if "name" not in self.state[p]:
                self.state[p]["name"] = self._param_names.get(p, "none")
        for pid, tensors in saved.items():
            p = id_map.get(pid)
            if p is None:
                continue
            st = self.state[p]
            # torch casts floating state to the parameter's dtype; restore the
            # saved tensor instead (a cast back would keep the bf16 rounding)
            for k, v in tensors.items():
                if torch.is_tensor(st.get(k)) and st[k].dtype != v.dtype:
                    st[k] = v.to(device=st[k].device, dtype=v.dtype)
            for k in _COUNTER_KEYS:  # counters follow this optimizer's capturable mode (gefen.py:5680-5705)
                if k in st:
                    v = st[k].item() if torch.is_tensor(st[k]) else st[k]
                    st[k] = self._new_step_counter(p.device, v)
        if global_step is not None:
            self._gefen_global_step = int(global_step)
        if self._capt_on:
            self._reset_gefen_global_step_devices()
        # The codebook is assigned unconditionally (gefen.py:5632-5641): a
        # checkpoint without one (taken before step 1) clears any stale
        # codebook, so the next step learns it again instead of skipping step 1.
        if codebook is not None:
            dev = next((p.device for g in self.param_groups for p in g["params"]), torch.device("cpu"))
            codebook = codebook.to(device=dev, dtype=torch.float32)
        self._gefen_codebook = codebook
        self._gefen_codebook_by_device.clear()
