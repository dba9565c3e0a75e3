"""Host logic of the GradScaler protocol (reference gefen.py:614-707, 853-894):
control parsing, the overflow skip, the in-place unscale and the protocol
choice. CPU tensors only; no kernel runs."""
import types
import warnings

import pytest
import torch

from gefen.gefen import _amp_gate, _amp_native_scaling_required, _amp_prepare_step, _amp_step_controls


def _opt(*grads, **attrs):
    params = []
    for g in grads:
        p = torch.nn.Parameter(torch.zeros_like(g))
        p.grad = g.clone()
        params.append(p)
    o = types.SimpleNamespace(param_groups=[{"params": params}])
    for k, v in attrs.items():
        setattr(o, k, v)
    return o, params


def test_no_controls_is_an_ordinary_step():
    o, params = _opt(torch.ones(4))
    assert _amp_gate(o)
    assert torch.equal(params[0].grad, torch.ones(4))


def test_overflow_skips_without_touching_gradients():
    o, params = _opt(torch.full((4,), 64.0), found_inf=torch.ones(()), grad_scale=torch.tensor(64.0))
    assert not _amp_gate(o)
    assert torch.equal(params[0].grad, torch.full((4,), 64.0))


def test_finite_step_unscales_each_dtype_once():
    g32 = torch.tensor([3.0, -6.0, 0.5, 1e-3]) * 1024.0
    g16 = g32.to(torch.float16)
    o, params = _opt(g32, g16, found_inf=torch.zeros(()), grad_scale=torch.tensor(1024.0))
    assert _amp_prepare_step(o)
    assert torch.equal(params[0].grad, g32 / 1024.0)
    assert torch.equal(params[1].grad, (g16.float() * (1.0 / 1024.0)).to(torch.float16))


def test_non_power_of_two_scale_uses_the_fp64_reciprocal_rounded_to_fp32():
    scale = 3.0
    inv = torch.tensor(scale, dtype=torch.float64).reciprocal().float()
    g = torch.linspace(-5.0, 5.0, 11)
    o, params = _opt(g, found_inf=0.0, grad_scale=scale)
    assert _amp_prepare_step(o)
    assert torch.equal(params[0].grad, g * inv)


def test_manual_unscale_stage_leaves_gradients_alone():
    o, params = _opt(torch.full((3,), 5.0), found_inf=torch.zeros(()), grad_scale=None)
    assert _amp_gate(o)
    assert torch.equal(params[0].grad, torch.full((3,), 5.0))


@pytest.mark.parametrize("attrs,msg", [
    ({"found_inf": torch.zeros(2)}, "non-scalar found_inf"),
    ({"grad_scale": torch.ones(2)}, "non-scalar grad_scale"),
    ({"grad_scale": torch.tensor(float("inf"))}, "non-finite or non-positive"),
    ({"grad_scale": 0.0}, "non-finite or non-positive"),
    ({"grad_scale": -2.0}, "non-finite or non-positive"),
])
def test_malformed_controls_raise(attrs, msg):
    o, _ = _opt(torch.ones(2), **attrs)
    with pytest.raises(RuntimeError, match=msg):
        _amp_step_controls(o)


def test_protocol_choice_follows_fp16_gradients():
    o, _ = _opt(torch.ones(2), torch.ones(2, dtype=torch.bfloat16))
    assert not _amp_native_scaling_required(o)
    o, params = _opt(torch.ones(2), torch.ones(2, dtype=torch.float16))
    assert _amp_native_scaling_required(o)
    params[1].grad = None
    assert not _amp_native_scaling_required(o)


def test_fsdp1_flat_fp16_declines_native_protocol_with_one_warning():
    o, params = _opt(torch.ones(2, dtype=torch.float16))
    params[0]._is_flat_param = True
    with warnings.catch_warnings(record=True) as w:
        warnings.simplefilter("always")
        assert not _amp_native_scaling_required(o)
        assert not _amp_native_scaling_required(o)
    assert sum("ShardedGradScaler" in str(x.message) for x in w) == 1
