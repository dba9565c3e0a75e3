"""Constructor and param-group contract of the drop-in classes on the host
(the behaviour the reference's own host tests hold its classes to:
tests/test_validation_cpu.py, tests/test_core_correctness_cpu.py,
tests/test_epsilon_muon_param_group_cpu.py there): invalid hyperparameters
and parameters raise before anything is registered, add_param_group is all
or nothing, and the accepted input forms build the same groups."""
import math

import pytest
import torch
import torch.nn as nn

from gefen import Gefen, GefenMuon, GefenMuonHybrid


def _p1():
    return [("b", nn.Parameter(torch.randn(8)))]


def _p2():
    return [("w", nn.Parameter(torch.randn(8, 8)))]


@pytest.mark.parametrize("kwargs", [{"lr": -1.0}, {"betas": (1.0, 0.999)}, {"betas": (0.9, 1.0)},
                                    {"weight_decay": -0.1}, {"codebook_refresh_every": -1},
                                    {"eps": 0.0}, {"eps": -1e-8}, {"eps": math.inf}, {"eps": math.nan}])
def test_gefen_rejects_bad_hyperparams(kwargs):
    with pytest.raises(ValueError):
        Gefen(_p1(), **kwargs)


def test_gefen_rejects_capturable_with_codebook_refresh():
    with pytest.raises(ValueError):
        Gefen(_p1(), capturable=True, codebook_refresh_every=10)


def test_gefen_rejects_non_tensor_param():
    with pytest.raises(TypeError):
        Gefen([("bad", "not a tensor")])


def test_multi_element_tensor_lr_rejected():
    with pytest.raises(ValueError):
        Gefen(_p1(), lr=torch.tensor([1e-3, 2e-3]))


def test_complex_param_rejected_at_construction_and_add():
    with pytest.raises(ValueError):
        Gefen([("c", nn.Parameter(torch.randn(4, dtype=torch.complex64)))])
    opt = Gefen(_p1())
    with pytest.raises(ValueError):
        opt.add_param_group({"params": [("c", nn.Parameter(torch.randn(4, dtype=torch.complex64)))]})


def test_add_param_group_is_all_or_nothing():
    opt = Gefen(_p1())
    before = len(opt.param_groups)
    good = nn.Parameter(torch.randn(4))
    bad = nn.Parameter(torch.randn(4, dtype=torch.complex64))
    with pytest.raises(ValueError):
        opt.add_param_group({"params": [("good", good), ("bad", bad)]})
    assert len(opt.param_groups) == before
    assert not any(good is p for g in opt.param_groups for p in g["params"])
    dup = nn.Parameter(torch.randn(4))
    with pytest.raises(ValueError):
        opt.add_param_group({"params": [("a", dup), ("b", dup)]})
    assert len(opt.param_groups) == before


def test_add_param_group_error_paths():
    opt = Gefen(_p1())
    before = len(opt.param_groups)
    with pytest.raises(TypeError, match="param_group must be a dict"):
        opt.add_param_group([nn.Parameter(torch.randn(4))])
    with pytest.raises(ValueError, match="missing the 'params' key"):
        opt.add_param_group({"lr": 1e-3})
    with pytest.raises(ValueError, match="empty parameter list"):
        opt.add_param_group({"params": []})
    assert len(opt.param_groups) == before


def test_constructor_input_forms():
    bare = nn.Parameter(torch.randn(4, 4))
    opt = Gefen(bare, lr=1e-3)
    assert len(opt.param_groups) == 1 and opt.param_groups[0]["params"] == [bare]
    model = nn.Linear(4, 4)
    opt = Gefen((p for p in model.parameters()), lr=1e-3)
    assert len(opt.param_groups[0]["params"]) == 2
    opt = Gefen(list(model.named_parameters()), lr=1e-3)
    assert len(opt.param_groups[0]["params"]) == 2
    opt = Gefen([{"params": [model.weight], "lr": 1e-2}, {"params": [model.bias]}], lr=1e-3)
    assert [g["lr"] for g in opt.param_groups] == [1e-2, 1e-3]
    with pytest.raises(ValueError, match="empty parameter list"):
        Gefen([], lr=1e-3)


def test_add_param_group_fills_defaults():
    opt = Gefen(_p1(), lr=1e-3, betas=(0.8, 0.99), eps=1e-6, weight_decay=0.02)
    opt.add_param_group({"params": [("x", nn.Parameter(torch.randn(3)))], "lr": 5e-3})
    g = opt.param_groups[-1]
    assert g["lr"] == 5e-3 and g["weight_decay"] == 0.02 and g["eps"] == 1e-6


@pytest.mark.parametrize("kwargs", [{"lr": -1.0}, {"momentum": -0.5}, {"weight_decay": -0.1},
                                    {"adjust_lr_fn": "bogus"}, {"sharded_mode": "bogus"},
                                    {"normuon": True, "normuon_beta2": 1.0}, {"ns_schedule": "bogus"},
                                    {"eps": 0.0}, {"normuon_eps": 0.0}, {"eps": math.nan}])
def test_gefen_muon_rejects_bad_hyperparams(kwargs):
    with pytest.raises(ValueError):
        GefenMuon(_p2(), **kwargs)


def test_gefen_muon_rejects_non_2d_param():
    with pytest.raises(ValueError):
        GefenMuon([("b", nn.Parameter(torch.randn(8)))])
    opt = GefenMuon(_p2())
    before = len(opt.param_groups)
    with pytest.raises(ValueError):
        opt.add_param_group({"params": [("ok", nn.Parameter(torch.randn(4, 4))), ("b", nn.Parameter(torch.randn(4)))]})
    assert len(opt.param_groups) == before


@pytest.mark.parametrize("ns_steps", [0, -1, 100])
def test_gefen_muon_rejects_bad_ns_steps(ns_steps):
    with pytest.raises(ValueError):
        GefenMuon(_p2(), ns_steps=ns_steps)


def test_gefen_muon_add_param_group_fills_muon_options():
    opt = GefenMuon(_p2(), lr=0.02, momentum=0.9, nesterov=False, normuon=True)
    opt.add_param_group({"params": [("w2", nn.Parameter(torch.randn(4, 6)))], "lr": 0.01})
    g = opt.param_groups[-1]
    assert g["lr"] == 0.01 and g["momentum"] == 0.9 and g["nesterov"] is False and g["normuon"] is True


def test_hybrid_rejects_empty_params_and_add_param_group():
    with pytest.raises(ValueError):
        GefenMuonHybrid([], [], lr=1e-3)
    opt = GefenMuonHybrid(_p2(), _p1(), lr=1e-3)
    with pytest.raises(NotImplementedError):
        opt.add_param_group({"params": [nn.Parameter(torch.randn(4, 4))]})


def test_package_surface():
    """The names the reference package exports (src/gefen/__init__.py:10-21)
    that belong to the step: the optimizers, the split helpers, the kernels
    module and the version string (the distributed-checkpoint classes are
    not part of this build)."""
    import gefen
    for name in ("Gefen", "GefenMuon", "GefenMuonHybrid", "split_params_for_muon", "validate_split", "kernels",
                 "__version__"):
        assert name in gefen.__all__ and hasattr(gefen, name), name
    assert isinstance(gefen.__version__, str) and gefen.__version__
    assert hasattr(gefen.kernels, "automatic_gefen_fused")
