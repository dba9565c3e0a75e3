"""State colocation logic on the host (no GPU needed).

Gefen._colocate_param_state_ (reference gefen.py:1897-1927) moves the state
tensors of a parameter paged to another device; on a same-device step it must
not touch anything.  The "meta" device stands in for a second device here.
"""
import pytest
import torch

from gefen import Gefen
from gefen.gefen import _COLOCATABLE_STATE_KEYS


def _host_state():
    return {"name": "w", "automatic_period": 16, "step": 3, "factored_step": 3,
            "m_codebook": torch.zeros(4, 16, dtype=torch.uint8),
            "m_magnitude": torch.ones(4, 1), "v_row": torch.ones(8), "v_col": torch.ones(8),
            "other": torch.ones(2)}


def _opt(**kw):
    return Gefen([("w", torch.nn.Parameter(torch.zeros(8, 8)))], lr=1e-3, **kw)


def test_same_device_is_a_no_op():
    opt = _opt()
    st = _host_state()
    before = dict(st)
    opt._colocate_param_state_(st, torch.device("cpu"))
    for k, v in before.items():
        assert st[k] is v, k


def test_moves_every_state_tensor_and_nothing_else():
    opt = _opt()
    st = _host_state()
    opt._colocate_param_state_(st, torch.device("meta"))
    for k in ("m_codebook", "m_magnitude", "v_row", "v_col"):
        assert st[k].device.type == "meta", k
        assert k in _COLOCATABLE_STATE_KEYS
    assert st["other"].device.type == "cpu"  # not optimizer state of the step
    assert st["automatic_period"] == 16 and st["step"] == 3 and st["name"] == "w"


def test_capturable_never_moves_state():
    opt = _opt(capturable=True)
    st = _host_state()
    before = dict(st)
    opt._colocate_param_state_(st, torch.device("meta"))
    for k, v in before.items():
        assert st[k] is v, k


def test_no_state_yet_is_a_no_op():
    opt = _opt()
    st = {"name": "w"}
    opt._colocate_param_state_(st, torch.device("meta"))
    assert st == {"name": "w"}


@pytest.mark.skipif(torch.cuda.is_available(), reason="host parameters are stepped when a HIP device exists")
def test_host_parameters_without_a_hip_device_are_refused():
    """Host-resident parameters are stepped on a HIP device through pinned
    staging; with none available the step refuses before anything mutates
    (there is no host arithmetic in the product)."""
    p = torch.nn.Parameter(torch.randn(16, 16))
    opt = Gefen([("w", p)], lr=1e-2, fused=False)
    assert opt.fused is False
    p.grad = torch.randn(16, 16) * 0.1
    with pytest.raises(RuntimeError, match="on a HIP device, and none is available"):
        opt.step()
    assert opt._gefen_codebook is None
    assert "automatic_period" not in opt.state.get(p, {})


def test_capturable_host_parameters_are_refused():
    p = torch.nn.Parameter(torch.randn(16, 16))
    opt = Gefen([("w", p)], lr=1e-2, capturable=True)
    p.grad = torch.randn(16, 16) * 0.1
    with pytest.raises(RuntimeError, match="capturable=True steps HIP device parameters only"):
        opt.step()
    assert opt._gefen_codebook is None
