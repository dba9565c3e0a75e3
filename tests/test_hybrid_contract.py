"""Drop-in construction contract of GefenMuonHybrid and Gefen's groups on the
host (no step: the product steps on the GPU only).  The reference holds its
optimizers to these in tests/test_hybrid_ctor_and_lrcache_cpu.py; the stepping
half of that file is tests/test_gpu_hybrid_contract.py."""
import pytest
import torch
import torch.nn as nn

from gefen import Gefen, GefenMuon, GefenMuonHybrid
from gefen.gefen_muon import BATCHED_NS_DEFAULT_WORKSPACE_BYTES


def _names(groups):
    return {n for g in groups for n in g.get("param_names", ())}


class TinyLM(nn.Module):
    def __init__(self, vocab=32, dim=16):
        super().__init__()
        self.embed = nn.Embedding(vocab, dim)
        self.hidden = nn.Linear(dim, dim, bias=True)
        self.norm = nn.LayerNorm(dim)
        self.lm_head = nn.Linear(dim, vocab, bias=False)


def test_module_first_arg_routes_by_name_and_shape():
    model = TinyLM()
    opt = GefenMuonHybrid(model, lr=1e-3)
    muon, backup = _names(opt.muon.param_groups), _names(opt.backup.param_groups)
    assert any("hidden.weight" in n for n in muon)
    assert any("embed" in n for n in backup) and any("lm_head" in n for n in backup)
    assert not any("embed" in n or "lm_head" in n for n in muon)
    assert len(opt.muon.param_groups) == 1 and len(opt.backup.param_groups) == 1
    assert len(opt.param_groups) == 2
    assert sum(len(g["params"]) for g in opt.param_groups) == sum(1 for _ in model.parameters())


def test_named_params_iterable_and_two_list_forms():
    model = TinyLM()
    opt = GefenMuonHybrid(list(model.named_parameters()), lr=1e-3)
    assert any("embed" in n for n in _names(opt.backup.param_groups))
    muon = [("hidden.weight", model.hidden.weight)]
    backup = [(n, p) for n, p in model.named_parameters() if p is not model.hidden.weight]
    opt2 = GefenMuonHybrid(muon, backup, lr=1e-3)
    assert opt2.muon is not None and opt2.backup is not None


def test_bare_tensors_rejected():
    with pytest.raises(TypeError, match=r"can't be routed|Bare tensors"):
        GefenMuonHybrid(list(TinyLM().parameters()), lr=1e-3)


def test_backup_substrings_only_with_the_single_argument_form():
    model = TinyLM()
    with pytest.raises(TypeError, match="backup_substrings is only valid"):
        GefenMuonHybrid([("hidden.weight", model.hidden.weight)], [("norm.weight", model.norm.weight)], lr=1e-3,
                        backup_substrings=("embed",))
    opt = GefenMuonHybrid(model, lr=1e-3, backup_substrings=("embed", "lm_head", "hidden"))
    muon = _names(opt.muon.param_groups) if opt.muon else set()
    assert not any("hidden.weight" in n for n in muon)


def test_backup_optimizer_selector_names_and_repr():
    default = GefenMuonHybrid.from_model(TinyLM(), lr=1e-3)
    assert isinstance(default.backup, Gefen) and default.backup_optimizer == "gefen"
    model = TinyLM()
    adamw = GefenMuonHybrid.from_model(model, lr=1e-3, backup_optimizer="adamw")
    assert isinstance(adamw.backup, torch.optim.AdamW) and adamw.backup_optimizer == "adamw"
    assert _names(adamw.backup.param_groups) == {n for n, p in model.named_parameters() if p is not model.hidden.weight}
    r = repr(adamw)
    assert "muon_params=1" in r and "backup_params=5" in r and "backup_optimizer='adamw'" in r
    with pytest.raises(ValueError, match="backup_optimizer.*gefen.*adamw"):
        GefenMuonHybrid.from_model(TinyLM(), lr=1e-3, backup_optimizer="sgd")


@pytest.mark.parametrize(("fused", "capturable"), [(False, False), (True, True)])
def test_adamw_backup_forwards_execution_flags(fused, capturable):
    opt = GefenMuonHybrid([], [("bias", nn.Parameter(torch.ones(4)))], lr=1e-3, backup_optimizer="adamw",
                          fused=fused, capturable=capturable)
    g = opt.backup.param_groups[0]
    assert g["fused"] is fused and g["capturable"] is capturable


def test_batched_ns_options_reach_the_muon_child():
    opt = GefenMuonHybrid.from_model(TinyLM(), lr=1e-3, batched_ns=True, batched_ns_workspace_bytes=64 << 20)
    assert opt.muon._batched_ns is True and opt.muon._batched_ns_workspace_bytes == 64 << 20
    assert all(g["batched_ns"] is True and g["batched_ns_workspace_bytes"] == 64 << 20
               for g in opt.muon.param_groups)
    opt = GefenMuonHybrid.from_model(TinyLM(), lr=1e-3)
    assert opt.muon._batched_ns is False
    assert all(g["batched_ns"] is False and g["batched_ns_workspace_bytes"] == BATCHED_NS_DEFAULT_WORKSPACE_BYTES
               for g in opt.muon.param_groups)


def test_user_param_groups_are_kept():
    p0, p1, p2 = nn.Parameter(torch.randn(4, 4)), nn.Parameter(torch.randn(4)), nn.Parameter(torch.randn(4, 4))
    opt = Gefen([{"params": [("layer0.weight", p0), ("layer0.bias", p1)], "lr": 1e-3},
                 {"params": [("layer1.weight", p2)], "lr": 2e-3}])
    assert [len(g["params"]) for g in opt.param_groups] == [2, 1]
    assert opt.param_groups[0]["param_names"] == ["layer0.weight", "layer0.bias"]
    assert opt.param_groups[1]["param_names"] == ["layer1.weight"]
    assert len(opt.state_dict()["param_groups"]) == 2
    for g, lr in zip(opt.param_groups, [1e-4, 2e-4]):
        g["lr"] = lr
    assert [g["lr"] for g in opt.param_groups] == [1e-4, 2e-4]


def test_repeated_group_names_get_distinct_parameter_names():
    p0, p1, p2 = (nn.Parameter(torch.ones(2, 2)) for _ in range(3))
    opt = Gefen([{"params": [p0], "name": "dup"}], lr=1e-3)
    opt.add_param_group({"params": [p1], "name": "dup"})
    opt.add_param_group({"params": [p2], "name": "dup"})
    assert [g["param_names"] for g in opt.param_groups] == [["dup"], ["dup_1"], ["dup_2"]]


def test_lr_scalar_single_slot_contract():
    opt = Gefen(nn.Linear(8, 8).parameters(), lr=torch.tensor(1e-3))
    g = opt.param_groups[0]
    assert opt._lr_scalar(g) == pytest.approx(1e-3)
    cache = opt._lr_scalar_cache
    assert isinstance(cache, tuple) and len(cache) == 3
    g["lr"].mul_(2.0)
    assert opt._lr_scalar(g) == pytest.approx(2e-3)
    opt = Gefen(nn.Linear(8, 8).parameters(), lr=1e-3)
    assert opt._lr_scalar(opt.param_groups[0]) == 1e-3
    assert getattr(opt, "_lr_scalar_cache", None) is None
    assert GefenMuon._lr_scalar is Gefen._lr_scalar


class _FrozenLM(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed_tokens = nn.Embedding(32, 16)
        self.proj = nn.Linear(16, 16)
        self.norm = nn.LayerNorm(16)
        self.lm_head = nn.Linear(16, 32, bias=False)
        self.frozen = nn.Linear(16, 16)
        self.frozen.weight.requires_grad_(False)
        self.frozen.bias.requires_grad_(False)


def test_from_model_covers_every_trainable_parameter_and_only_those():
    model = _FrozenLM()
    opt = GefenMuonHybrid.from_model(model, lr=1e-3)
    assert {id(p) for g in opt.param_groups for p in g["params"]} == {id(p) for p in model.parameters()
                                                                       if p.requires_grad}


def test_per_half_lr_and_the_hybrid_surface():
    model = _FrozenLM()
    opt = GefenMuonHybrid.from_model(model, lr=1e-3, backup_lr=5e-4)
    lrs = {g["lr"] for g in opt.param_groups}
    assert 5e-4 in lrs and any(abs(lr - 5e-4) > 1e-12 for lr in lrs)
    with pytest.raises(NotImplementedError):
        opt.add_param_group({"params": [nn.Parameter(torch.randn(4, 4))]})
    with pytest.warns(UserWarning, match="adjust_lr_fn"):
        GefenMuonHybrid.from_model(_FrozenLM(), lr=1e-3, adjust_lr_fn=None)


def test_one_determinism_policy_reaches_both_gefen_children():
    opt = GefenMuonHybrid.from_model(nn.Sequential(nn.Linear(8, 8), nn.LayerNorm(8)), lr=1e-3,
                                     backup_optimizer="gefen", deterministic=True)
    assert opt._deterministic is True
    assert opt.muon is not None and opt.muon._deterministic is True
    assert opt.backup is not None and opt.backup._deterministic is True
    assert set(opt.state_dict()) == {"muon", "backup", "backup_optimizer"}


# ----------------------------------------------- ZeRO-3 placeholder guard
# (the reference's tests/test_zero_incompat_guard_cpu.py:163-205, 313-325)


def test_zero3_placeholders_refused_in_both_forms():
    placeholders = [("model.embed.weight", nn.Parameter(torch.empty(0))),
                    ("model.layers.0.mlp.w", nn.Parameter(torch.empty(0))),
                    ("model.norm.weight", nn.Parameter(torch.empty(0)))]
    with pytest.raises(ValueError, match="ZeRO stage 3") as info:
        GefenMuonHybrid(placeholders, lr=1e-3, fused=False)
    msg = str(info.value)
    assert "zero-numel" in msg and "backup-only" in msg and "plain Gefen" in msg
    with pytest.raises(ValueError, match="ZeRO stage 3"):
        GefenMuonHybrid([], [("model.norm.weight", nn.Parameter(torch.empty(0)))], lr=1e-3, fused=False)


def test_real_or_mixed_backup_only_sets_still_construct():
    real = [("norm.weight", nn.Parameter(torch.randn(8))), ("norm.bias", nn.Parameter(torch.randn(8)))]
    opt = GefenMuonHybrid([], real, lr=1e-3)
    assert opt.muon is None and isinstance(opt.backup, Gefen)
    mixed = [("real.weight", nn.Parameter(torch.zeros(8))), ("empty.slot", nn.Parameter(torch.zeros(0)))]
    opt = GefenMuonHybrid([], mixed, lr=1e-3)
    assert opt.muon is None and len(opt.param_groups) == 1
    with pytest.raises(ValueError, match="no parameters"):
        GefenMuonHybrid([], [], lr=1e-3)


# ------------------------------------------------- backup group cohorts


@pytest.mark.parametrize("backup", ["gefen", "adamw"])
def test_no_decay_cohorts(backup):
    model = TinyLM()
    opt = GefenMuonHybrid.from_model(model, lr=1e-3, backup_lr=4e-4, backup_weight_decay=0.1,
                                     weight_decay=0.05, betas=(0.8, 0.99), eps=1e-7,
                                     no_decay_substrings=("NORM", "bias"), backup_optimizer=backup)
    groups = opt.backup.param_groups
    assert len(groups) == 2
    decay, exempt = groups
    assert set(decay["param_names"]) == {"embed.weight", "lm_head.weight"}
    assert set(exempt["param_names"]) == {"hidden.bias", "norm.weight", "norm.bias"}
    assert decay["weight_decay"] == 0.1 and exempt["weight_decay"] == 0.0
    for g in groups:
        assert g["lr"] == 4e-4 and g["eps"] == 1e-7
        if backup == "adamw":
            assert tuple(g["betas"]) == (0.8, 0.99)
        else:
            assert (g["beta1"], g["beta2"]) == (0.8, 0.99)
    # the Muon half keeps the shared weight decay
    assert all(g["weight_decay"] == 0.05 for g in opt.muon.param_groups)
    # a substring no name contains leaves one decaying cohort (the empty one is dropped)
    opt = GefenMuonHybrid.from_model(TinyLM(), lr=1e-3, weight_decay=0.05, no_decay_substrings=("zzz",),
                                     backup_optimizer=backup)
    assert len(opt.backup.param_groups) == 1 and opt.backup.param_groups[0]["weight_decay"] == 0.05


@pytest.mark.parametrize("backup", ["gefen", "adamw"])
def test_without_no_decay_one_default_group(backup):
    opt = GefenMuonHybrid.from_model(TinyLM(), lr=2e-3, weight_decay=0.02, backup_optimizer=backup)
    (g,) = opt.backup.param_groups
    assert g["lr"] == 2e-3 and g["weight_decay"] == 0.02
    assert opt.backup.defaults["lr"] == 2e-3 and opt.backup.defaults["weight_decay"] == 0.02
    if backup == "gefen":
        assert opt.backup._factored_v_2d is False


# ------------------------------------ load: the shadow runs child pre-hooks


def test_adamw_child_pre_hook_can_migrate_a_checkpoint():
    """A checkpoint the AdamW child's own load pre-hook repairs (a missing
    "step" added back) loads through the hybrid's preflight."""
    p = nn.Parameter(torch.randn(6))
    opt = GefenMuonHybrid([], [("bias", p)], lr=1e-3, backup_optimizer="adamw", fused=False)
    p.grad = torch.full_like(p, 1e-3)
    opt.backup.step()
    ckpt = opt.state_dict()
    del ckpt["backup"]["state"][0]["step"]

    def add_step(child, sd):
        for st in sd["state"].values():
            st.setdefault("step", torch.tensor(1.0))
        return sd

    fresh_p = nn.Parameter(torch.randn(6))
    fresh = GefenMuonHybrid([], [("bias", fresh_p)], lr=1e-3, backup_optimizer="adamw", fused=False)
    with pytest.raises(KeyError, match="step"):
        fresh.load_state_dict(ckpt)
    assert not fresh.backup.state
    fresh.backup.register_load_state_dict_pre_hook(add_step)
    fresh.load_state_dict(ckpt)
    assert float(fresh.backup.state[fresh_p]["step"]) == 1.0
    assert torch.equal(fresh.backup.state[fresh_p]["exp_avg"], opt.backup.state[p]["exp_avg"])
