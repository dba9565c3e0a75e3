"""The Muon quality levers as the reference checks them on a GPU
(tests/test_muon_quality_levers.py there): with the flags off no lever state
exists and stepping is repeatable; NorMuon changes the trajectory, keeps
[rows, 1] fp32 state that survives a state_dict round trip, and preserves the
Frobenius norm of the update in both orientations; the cautious mask zeroes
exactly the disagreeing coordinates and rescales the rest by bf16(numel /
agree); cautious stepping changes the trajectory without NorMuon state."""
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _run(dev, seed=0, n=4, shape=(256, 512), **kw):
    from gefen import GefenMuon
    torch.manual_seed(seed)
    p = (torch.randn(*shape, device=dev) * 0.02).bfloat16().requires_grad_()
    opt = GefenMuon([("w", p)], lr=1e-3, adjust_lr_fn="match_rms_adamw", **kw)
    torch.manual_seed(seed + 1)
    for _ in range(n):
        p.grad = torch.randn(*shape, device=dev).bfloat16() * 1e-3
        opt.step()
    torch.cuda.synchronize()
    return p.detach().clone(), opt


def test_flags_off_no_lever_state_and_repeatable(dev):
    p1, opt1 = _run(dev)
    p2, _ = _run(dev)
    assert torch.equal(p1, p2)
    st = next(iter(opt1.state.values()))
    assert "normuon_v" not in st and "normuon_step" not in st


def test_normuon_engages_with_row_state(dev):
    base, _ = _run(dev)
    nm, opt = _run(dev, normuon=True)
    assert not torch.equal(base, nm) and torch.isfinite(nm).all()
    st = next(iter(opt.state.values()))
    assert st["normuon_v"].dtype == torch.float32 and tuple(st["normuon_v"].shape) == (256, 1)
    assert st["normuon_step"] == 4


@pytest.mark.parametrize("shape", [(256, 1024), (1024, 256)])
def test_normuon_preserves_the_frobenius_norm(dev, shape):
    from gefen import GefenMuon
    opt = GefenMuon([("w", torch.zeros(4, 4, device=dev).bfloat16().requires_grad_())], lr=1e-3, normuon=True)
    for _ in range(3):
        o = torch.randn(*shape, device=dev).bfloat16()
        out = opt._normuon_normalize({}, o.clone(), 0.95, 1e-8)
        n_in, n_out = o.float().norm().item(), out.float().norm().item()
        assert abs(n_in - n_out) / n_in < 5e-3, (shape, n_in, n_out)


def test_normuon_state_round_trips(dev):
    _, opt = _run(dev, normuon=True)
    sd = opt.state_dict()
    _, opt3 = _run(dev, normuon=True, seed=99)
    assert not torch.equal(next(iter(opt3.state.values()))["normuon_v"], next(iter(opt.state.values()))["normuon_v"])
    opt3.load_state_dict(sd)
    old, new = next(iter(opt.state.values())), next(iter(opt3.state.values()))
    assert new["normuon_v"].dtype == torch.float32 and torch.equal(new["normuon_v"], old["normuon_v"])
    assert new["normuon_step"] == old["normuon_step"]


def test_cautious_mask_helper_property(dev):
    from gefen.gefen_muon import _cautious_mask_
    torch.manual_seed(0)
    u = torch.randn(128, 256, device=dev).bfloat16()
    g = torch.randn(128, 256, device=dev).bfloat16()
    out = _cautious_mask_(u.clone(), g)
    agree = (u * g) > 0
    assert (out[~agree] == 0).all()
    scale = agree.numel() / agree.sum().float()
    assert torch.equal(out[agree], (u[agree].float() * scale.to(torch.bfloat16).float()).bfloat16())


def test_cautious_engages_without_normuon_state(dev):
    base, _ = _run(dev)
    ca, opt = _run(dev, cautious=True)
    assert not torch.equal(base, ca) and torch.isfinite(ca).all()
    assert "normuon_v" not in next(iter(opt.state.values()))
