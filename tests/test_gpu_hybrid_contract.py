"""Stepping half of the drop-in contract the reference holds GefenMuonHybrid
and Gefen's groups to (tests/test_hybrid_ctor_and_lrcache_cpu.py there), on
MI355X: every construction form steps; an AdamW backup equals a standalone
torch AdamW built from the same named groups, bit for bit; an LR scheduler
keeps the Muon/backup lr split; parameters sharing a name keep separate
state; per-group lr and weight decay route numerically."""
import warnings

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


def _step(opt, model, dev):
    gen = torch.Generator().manual_seed(3)
    idx = torch.randint(0, 32, (4, 6), generator=gen).to(dev)
    tgt = torch.randint(0, 32, (4, 6), generator=gen).to(dev)

    def closure():
        opt.zero_grad()
        loss = nn.functional.cross_entropy(model(idx).reshape(-1, 32), tgt.reshape(-1))
        loss.backward()
        return loss

    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        loss = opt.step(closure)
    torch.cuda.synchronize()
    return float(loss)


@pytest.mark.parametrize("form", ["module", "named", "two_lists"])
def test_every_construction_form_steps(dev, form):
    from gefen import GefenMuonHybrid
    torch.manual_seed(0)
    model = TinyLM().to(dev)
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    if form == "module":
        opt = GefenMuonHybrid(model, lr=1e-3)
    elif form == "named":
        opt = GefenMuonHybrid(list(model.named_parameters()), lr=1e-3)
    else:
        muon = [("hidden.weight", model.hidden.weight)]
        opt = GefenMuonHybrid(muon, [(n, p) for n, p in model.named_parameters() if p is not model.hidden.weight],
                              lr=1e-3)
    assert _step(opt, model, dev) > 0.0
    for n, p in model.named_parameters():
        assert torch.isfinite(p).all(), n
        assert not torch.equal(p, before[n]), n


def test_adamw_backup_equals_standalone_adamw(dev):
    from gefen import GefenMuonHybrid
    torch.manual_seed(13)
    w0, b0 = torch.randn(5, 3), torch.randn(5)
    hw, hb = nn.Parameter(w0.clone().to(dev)), nn.Parameter(b0.clone().to(dev))
    rw, rb = nn.Parameter(w0.clone().to(dev)), nn.Parameter(b0.clone().to(dev))
    lr, betas, eps, wd = 4e-4, (0.8, 0.95), 2e-7, 0.2
    opt = GefenMuonHybrid([], [("proj.weight", hw), ("norm.bias", hb)], lr=1e-3, backup_lr=lr,
                          backup_weight_decay=wd, backup_optimizer="adamw", no_decay_substrings=("bias",),
                          backup_1d_period_one=True, backup_2d_period_one=True, betas=betas, eps=eps, fused=False)
    ref = torch.optim.AdamW([{"params": [rw], "lr": lr, "betas": betas, "eps": eps, "weight_decay": wd},
                             {"params": [rb], "lr": lr, "betas": betas, "eps": eps, "weight_decay": 0.0}],
                            lr=lr, betas=betas, eps=eps, weight_decay=wd, fused=False)
    assert [g["param_names"] for g in opt.backup.param_groups] == [["proj.weight"], ["norm.bias"]]
    assert [g["weight_decay"] for g in opt.backup.param_groups] == [wd, 0.0]
    assert all(g["lr"] == lr and g["betas"] == betas and g["eps"] == eps for g in opt.backup.param_groups)
    gen = torch.Generator().manual_seed(19)
    for _ in range(4):
        gw, gb = torch.randn(5, 3, generator=gen).to(dev), torch.randn(5, generator=gen).to(dev)
        hw.grad, rw.grad, hb.grad, rb.grad = gw.clone(), gw.clone(), gb.clone(), gb.clone()
        opt.step()
        ref.step()
        opt.zero_grad()
        ref.zero_grad()
    torch.cuda.synchronize()
    assert torch.equal(hw, rw) and torch.equal(hb, rb)
    assert opt.backup.state[hw]["exp_avg_sq"].shape == hw.shape


def test_scheduler_keeps_the_lr_split(dev):
    from gefen import GefenMuonHybrid
    torch.manual_seed(0)
    model = TinyLM().to(dev)
    opt = GefenMuonHybrid.from_model(model, lr=1e-3, backup_lr=2.5e-4, backup_optimizer="adamw")
    sched = torch.optim.lr_scheduler.StepLR(opt, step_size=1, gamma=0.1)
    _step(opt, model, dev)
    sched.step()
    assert [g["lr"] for g in opt.muon.param_groups] == pytest.approx([1e-4])
    assert [g["lr"] for g in opt.backup.param_groups] == pytest.approx([2.5e-5])


def test_same_name_parameters_keep_separate_state(dev):
    from gefen import Gefen
    p0 = nn.Parameter(torch.ones(3, 3, device=dev))
    p1 = nn.Parameter(torch.ones(3, 3, device=dev) * 2.0)
    opt = Gefen([{"params": [("shared.weight", p0), ("shared.weight", p1)], "lr": 1e-3}])
    p0.grad = torch.full_like(p0, 0.01)
    p1.grad = torch.full_like(p1, -0.02)
    opt.step()
    torch.cuda.synchronize()
    assert opt.param_groups[0]["param_names"] == ["shared.weight", "shared.weight"]
    assert opt.state[p0] is not opt.state[p1]
    assert opt.state[p0]["name"] == opt.state[p1]["name"] == "shared.weight"
    assert opt.state[p0]["m_codebook"].data_ptr() != opt.state[p1]["m_codebook"].data_ptr()
    assert (p0 < 1.0).all() and (p1 > 2.0).all()  # each moved against its own gradient


def test_group_names_name_their_parameters_after_a_step(dev):
    from gefen import Gefen
    p0, p1, p2 = (nn.Parameter(torch.ones(2, 2, device=dev)) for _ in range(3))
    opt = Gefen([{"params": [p0], "name": "dup"}], lr=1e-3)
    opt.add_param_group({"params": [p1], "name": "dup"})
    opt.add_param_group({"params": [p2], "name": "dup"})
    for p in (p0, p1, p2):
        p.grad = torch.full_like(p, 0.01)
    opt.step()
    assert [opt.state[p]["name"] for p in (p0, p1, p2)] == ["dup", "dup_1", "dup_2"]


def test_per_group_lr_and_weight_decay_route_numerically(dev):
    from gefen import Gefen
    pn, pl, ph = (nn.Parameter(torch.ones(4, device=dev)) for _ in range(3))
    opt = Gefen([{"params": [("no_decay", pn)], "lr": 3e-2, "weight_decay": 0.0},
                 {"params": [("low_lr", pl)], "lr": 1e-2, "weight_decay": 0.1},
                 {"params": [("high_lr", ph)], "lr": 3e-2, "weight_decay": 0.1}], lr=1e-2, weight_decay=0.0)
    for p in (pn, pl, ph):
        p.grad = torch.zeros_like(p)
    opt.step()
    torch.cuda.synchronize()
    torch.testing.assert_close(pn, torch.ones_like(pn))
    torch.testing.assert_close(pl, torch.full_like(pl, 1.0 - 1e-2 * 0.1))
    torch.testing.assert_close(ph, torch.full_like(ph, 1.0 - 3e-2 * 0.1))
    assert (1.0 - ph).abs().mean().item() == pytest.approx(3.0 * (1.0 - pl).abs().mean().item(), rel=1e-4)
