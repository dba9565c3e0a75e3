"""GradScaler protocols on the GPU step (intent of the reference's
tests/test_amp_grad_scaler.py:309-457).

True fp16 gradients take the optimizer-side ("native") protocol: GradScaler
hands the optimizer ``found_inf`` and ``grad_scale``, a finite step unscales
in place and then steps exactly as an unscaled step would, and an overflow is a
complete no-op (parameters, state and state_dict bit-identical to before).
fp32-master and bf16 training keep GradScaler's ordinary path. Every step runs
the fused HIP kernels through libgefenx.so.
"""
import copy

import pytest
import torch
import torch.nn as nn

from gefen import Gefen, GefenMuon, GefenMuonHybrid

pytestmark = pytest.mark.gpu


class _Fp16ManualGradScaler(torch.amp.GradScaler):
    """GradScaler whose explicit unscale_ accepts fp16 gradients (the sharded
    scaler's behaviour), to stage a manual unscale before step."""

    def _unscale_grads_(self, optimizer, inv_scale, found_inf, allow_fp16):
        return super()._unscale_grads_(optimizer, inv_scale, found_inf, True)


def _values(seed, scale, dtype):
    gen = torch.Generator(device="cpu").manual_seed(seed)
    matrix = (torch.randn(32, 32, generator=gen) * scale).to("cuda", dtype)
    bias = (torch.randn(32, generator=gen) * scale).to("cuda", dtype)
    return matrix, bias


def _make(kind, dtype, backup_optimizer="gefen"):
    m0, b0 = _values(7101, 0.02, dtype)
    matrix = nn.Parameter(m0.clone())
    if kind == "gefen":
        return Gefen([("layer.weight", matrix)], lr=2e-3, fused=True, factored_v_2d=False), [matrix]
    if kind == "muon":
        return GefenMuon([("layer.weight", matrix)], lr=2e-3, fused=True, ns_steps=2,
                         ns_schedule="standard", adjust_lr_fn="original"), [matrix]
    bias = nn.Parameter(b0.clone())
    opt = GefenMuonHybrid([("layer.weight", matrix)], [("layer.bias", bias)], lr=2e-3, fused=True,
                          ns_steps=2, ns_schedule="standard", normuon=False,
                          backup_optimizer=backup_optimizer)
    return opt, [matrix, bias]


def _grads(kind, dtype):
    m, b = _values(7102, 0.002, dtype)
    return [m, b] if kind == "hybrid" else [m]


def _scaler(cls=torch.amp.GradScaler, scale=128.0):
    s = cls("cuda", init_scale=scale)
    s.scale(torch.ones((), device="cuda"))  # materialise the device scale
    return s


def _set_grads(params, grads, scale=None):
    for p, g in zip(params, grads):
        p.grad = g.clone() if scale is None else (g * scale).to(p.dtype)


def _clone(v):
    if torch.is_tensor(v):
        return v.detach().clone()
    if isinstance(v, dict):
        return {k: _clone(x) for k, x in v.items()}
    if isinstance(v, (list, tuple)):
        return type(v)(_clone(x) for x in v)
    return copy.deepcopy(v)


def _assert_same(a, b):
    if torch.is_tensor(b):
        assert torch.is_tensor(a) and a.dtype == b.dtype and a.device == b.device
        assert torch.equal(a, b)
    elif isinstance(b, dict):
        assert isinstance(a, dict) and set(a) == set(b)
        for k in b:
            _assert_same(a[k], b[k])
    elif isinstance(b, (list, tuple)):
        assert type(a) is type(b) and len(a) == len(b)
        for x, y in zip(a, b):
            _assert_same(x, y)
    else:
        assert a == b


KINDS = ["gefen", "muon", "hybrid"]


@pytest.mark.parametrize("kind", KINDS)
def test_finite_fp16_scaler_step_matches_unscaled_step(kind):
    ref, ref_params = _make(kind, torch.float16)
    opt, params = _make(kind, torch.float16)
    grads = _grads(kind, torch.float16)
    _set_grads(ref_params, grads)
    ref.step()

    scaler = _scaler()
    _set_grads(params, grads, scaler.get_scale())
    assert opt._step_supports_amp_scaling
    scaler.step(opt)
    scaler.update()
    torch.cuda.synchronize()
    for p, g in zip(params, grads):
        assert torch.equal(p.grad, g)  # unscaled in place, exactly (scale is a power of two)
    for a, b in zip(params, ref_params):
        assert torch.equal(a.detach(), b.detach())
    _assert_same(opt.state_dict(), ref.state_dict())


@pytest.mark.parametrize("initialized", [False, True], ids=["first_step", "initialized"])
@pytest.mark.parametrize("kind", KINDS)
def test_fp16_overflow_is_a_complete_noop(kind, initialized):
    opt, params = _make(kind, torch.float16)
    scaler = _scaler()
    grads = _grads(kind, torch.float16)
    if initialized:
        _set_grads(params, grads, scaler.get_scale())
        scaler.step(opt)
        scaler.update()
        opt.zero_grad(set_to_none=True)
    before_params = [p.detach().clone() for p in params]
    before_sd = _clone(opt.state_dict())
    _set_grads(params, grads, scaler.get_scale())
    params[0].grad.view(-1)[0] = float("inf")
    scale_before = scaler.get_scale()
    assert scaler.step(opt) is None
    scaler.update()
    torch.cuda.synchronize()
    assert scaler.get_scale() < scale_before
    for a, b in zip(params, before_params):
        assert torch.equal(a.detach(), b)
    _assert_same(opt.state_dict(), before_sd)


@pytest.mark.parametrize("kind", KINDS)
def test_fp32_manual_unscale_is_not_applied_twice(kind):
    ref, ref_params = _make(kind, torch.float32)
    opt, params = _make(kind, torch.float32)
    grads = _grads(kind, torch.float32)
    _set_grads(ref_params, [g * 0.25 for g in grads])
    ref.step()

    scaler = _scaler()
    assert not opt._step_supports_amp_scaling  # fp32 keeps GradScaler's ordinary path
    _set_grads(params, grads, scaler.get_scale())
    scaler.unscale_(opt)
    for p, g in zip(params, grads):
        assert torch.equal(p.grad, g)
        p.grad.mul_(0.25)  # e.g. clipping between unscale_ and step
    scaler.step(opt)
    scaler.update()
    for a, b in zip(params, ref_params):
        assert torch.equal(a.detach(), b.detach())
    _assert_same(opt.state_dict(), ref.state_dict())


@pytest.mark.parametrize("kind", KINDS)
def test_fp16_manual_unscale_stage_is_not_divided_twice(kind):
    ref, ref_params = _make(kind, torch.float16)
    opt, params = _make(kind, torch.float16)
    grads = _grads(kind, torch.float16)
    _set_grads(ref_params, [(g * 0.5).to(torch.float16) for g in grads])
    ref.step()

    scaler = _scaler(_Fp16ManualGradScaler)
    _set_grads(params, grads, scaler.get_scale())
    scaler.unscale_(opt)
    assert opt._step_supports_amp_scaling
    for p, g in zip(params, grads):
        assert torch.equal(p.grad, g)
        p.grad.mul_(0.5)
    scaler.step(opt)  # grad_scale arrives as None: no second division
    scaler.update()
    for a, b in zip(params, ref_params):
        assert torch.equal(a.detach(), b.detach())
    _assert_same(opt.state_dict(), ref.state_dict())


@pytest.mark.parametrize("overflow_half", ["muon", "backup"])
@pytest.mark.parametrize("initialized", [False, True], ids=["first_step", "initialized"])
def test_hybrid_overflow_in_one_half_skips_both_halves(initialized, overflow_half):
    opt, params = _make("hybrid", torch.float16, backup_optimizer="adamw")
    scaler = _scaler()
    grads = _grads("hybrid", torch.float16)
    if initialized:
        _set_grads(params, grads, scaler.get_scale())
        scaler.step(opt)
        scaler.update()
        opt.zero_grad(set_to_none=True)
    before_params = [p.detach().clone() for p in params]
    before_sd = _clone(opt.state_dict())
    _set_grads(params, grads, scaler.get_scale())
    params[0 if overflow_half == "muon" else 1].grad.view(-1)[0] = float("inf")
    scaler.step(opt)
    scaler.update()
    torch.cuda.synchronize()
    for a, b in zip(params, before_params):
        assert torch.equal(a.detach(), b)
    _assert_same(opt.state_dict(), before_sd)


@pytest.mark.parametrize("kind", KINDS)
def test_bf16_stays_on_the_ordinary_optimizer_path(kind):
    opt, params = _make(kind, torch.bfloat16)
    grads = _grads(kind, torch.bfloat16)
    assert not opt._step_supports_amp_scaling
    before = [p.detach().clone() for p in params]
    _set_grads(params, grads)
    opt.step()
    assert any(not torch.equal(p.detach(), b) for p, b in zip(params, before))
