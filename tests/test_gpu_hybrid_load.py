"""GefenMuonHybrid.load_state_dict fails before it mutates, on MI355X
(tests/test_hybrid_load_atomicity.py in the reference): a backup half that
either child loader would refuse leaves both children untouched and never
loads the Muon half; an AdamW backup whose checkpoint lacks "step" (torch
raises only after replacing its state) leaves both children untouched; a
child load post-hook that raises runs only after both halves are committed."""
import copy

import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


class TinyLM(nn.Module):
    def __init__(self, vocab=32, dim=16):
        super().__init__()
        self.embed = nn.Embedding(vocab, dim)
        self.hidden = nn.Linear(dim, dim, bias=True)
        self.norm = nn.LayerNorm(dim)
        self.lm_head = nn.Linear(dim, vocab, bias=False)

    def forward(self, idx):
        return self.lm_head(self.norm(self.hidden(self.embed(idx))))


def _build(dev, backup="gefen"):
    from gefen import GefenMuonHybrid
    torch.manual_seed(0)
    model = TinyLM().to(dev)
    return GefenMuonHybrid(model, lr=1e-3, backup_optimizer=backup), model


def _step(opt, model, dev):
    idx = torch.randint(0, 32, (4, 6), device=dev)
    tgt = torch.randint(0, 32, (4, 6), device=dev)
    opt.zero_grad()
    nn.functional.cross_entropy(model(idx).reshape(-1, 32), tgt.reshape(-1)).backward()
    opt.step()
    torch.cuda.synchronize()


def _snapshot(child):
    return {(id(p), k): (v.detach().clone(), id(v)) for p, st in child.state.items() for k, v in st.items()
            if torch.is_tensor(v)}


def _unchanged(child, before):
    after = _snapshot(child)
    assert set(after) == set(before)
    for k, (v, i) in before.items():
        assert torch.equal(after[k][0], v) and after[k][1] == i, k


@pytest.mark.parametrize("backup", ["gefen", "adamw"])
def test_backup_refusal_never_loads_the_muon_half(dev, backup):
    opt, model = _build(dev, backup)
    _step(opt, model, dev)
    bad = copy.deepcopy(opt.state_dict())
    bad["backup"]["param_groups"].append(copy.deepcopy(bad["backup"]["param_groups"][0]))
    muon_before, backup_before = _snapshot(opt.muon), _snapshot(opt.backup)
    calls = {"n": 0}
    load = opt.muon.load_state_dict

    def counting(sd):
        calls["n"] += 1
        return load(sd)

    opt.muon.load_state_dict = counting
    with pytest.raises(ValueError, match="different number of parameter groups"):
        opt.load_state_dict(bad)
    assert calls["n"] == 0
    _unchanged(opt.muon, muon_before)
    _unchanged(opt.backup, backup_before)


def test_adamw_backup_without_step_leaves_both_halves_untouched(dev):
    opt, model = _build(dev, "adamw")
    _step(opt, model, dev)
    _step(opt, model, dev)
    bad = copy.deepcopy(opt.state_dict())
    first = next(iter(bad["backup"]["state"]))
    del bad["backup"]["state"][first]["step"]
    muon_before, backup_before = _snapshot(opt.muon), _snapshot(opt.backup)
    with pytest.raises(KeyError, match="step"):
        opt.load_state_dict(bad)
    _unchanged(opt.muon, muon_before)
    _unchanged(opt.backup, backup_before)


@pytest.mark.parametrize("backup", ["gefen", "adamw"])
def test_raising_post_hook_runs_after_both_halves_commit(dev, backup):
    src, src_model = _build(dev, backup)
    for _ in range(3):
        _step(src, src_model, dev)
    ckpt = src.state_dict()
    want_muon = next(float(v["step"]) for v in src.muon.state.values() if "step" in v)
    want_backup = next(float(v["step"]) for v in src.backup.state.values() if "step" in v)
    opt, model = _build(dev, backup)
    _step(opt, model, dev)

    def boom(_):
        raise RuntimeError("post-hook boom")

    opt.muon.register_load_state_dict_post_hook(boom)
    with pytest.raises(RuntimeError, match="post-hook boom"):
        opt.load_state_dict(ckpt)
    assert next(float(v["step"]) for v in opt.muon.state.values() if "step" in v) == want_muon
    assert next(float(v["step"]) for v in opt.backup.state.values() if "step" in v) == want_backup
