"""Step-level contract on MI355X that the reference's host tests hold its
step to (tests/test_core_correctness_cpu.py there): a frozen parameter stays
registered, is skipped while it has no grad and trains once unfrozen; a
stale legacy state key is inert on load; sparse and complex grads are
refused cleanly before anything moves; fp16 grads whose squares overflow
fp16 give a finite second moment (the squares are taken in fp32)."""
import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def test_frozen_param_registered_then_trains(dev):
    from gefen import Gefen
    torch.manual_seed(0)
    lin, frozen = nn.Linear(64, 64).to(dev), nn.Linear(64, 64).to(dev)
    frozen.weight.requires_grad_(False)
    frozen.bias.requires_grad_(False)
    opt = Gefen(list(lin.named_parameters()) + [("frozen." + n, p) for n, p in frozen.named_parameters()], lr=1e-2)
    assert {id(frozen.weight), id(frozen.bias)} <= {id(p) for g in opt.param_groups for p in g["params"]}
    lin.weight.grad = torch.randn_like(lin.weight) * 0.1
    lin.bias.grad = torch.randn_like(lin.bias) * 0.1
    before = frozen.weight.detach().clone()
    opt.step()
    assert torch.equal(before, frozen.weight) and "step" not in opt.state.get(frozen.weight, {})
    frozen.weight.requires_grad_(True)
    frozen.weight.grad = torch.randn_like(frozen.weight) * 0.1
    opt.step()
    torch.cuda.synchronize()
    assert not torch.equal(before, frozen.weight) and torch.isfinite(frozen.weight).all()


def test_legacy_state_key_is_inert(dev):
    from gefen import Gefen

    def make():
        torch.manual_seed(0)
        model = nn.Linear(32, 32).to(dev)
        return model, Gefen(list(model.named_parameters()), lr=1e-2)

    model, opt = make()
    for p in model.parameters():
        p.grad = torch.randn_like(p) * 0.1
    opt.step()
    sd = opt.state_dict()
    for st in sd["state"].values():
        st["m_codebook_shape"] = tuple(st["m_codebook"].shape)
    model2, opt2 = make()
    opt2.load_state_dict(sd)
    for p in model2.parameters():
        p.grad = torch.randn_like(p) * 0.1
    opt2.step()
    torch.cuda.synchronize()
    assert all(torch.isfinite(p).all() for p in model2.parameters())


def test_sparse_and_complex_grads_refused_before_any_mutation(dev):
    from gefen import Gefen
    p = nn.Parameter(torch.randn(4, 4, device=dev))
    q = nn.Parameter(torch.randn(8, device=dev))
    opt = Gefen([("q", q), ("p", p)], lr=1e-2)
    q.grad = torch.randn_like(q)
    p.grad = torch.sparse_coo_tensor(torch.tensor([[0, 1], [0, 1]]), torch.tensor([1.0, 2.0]), (4, 4)).to(dev)
    q0 = q.detach().clone()
    with pytest.raises(RuntimeError, match="sparse gradient"):
        opt.step()
    assert opt._gefen_codebook is None and torch.equal(q0, q)


def test_fp16_vmean_does_not_overflow(dev):
    from gefen.kernels.automatic_vmean import automatic_vmean_update_cuda
    vmean = torch.zeros(2, 1, dtype=torch.float32, device=dev)
    g = torch.full((2, 8), 300.0, dtype=torch.float16, device=dev)  # 300^2 > fp16 max
    automatic_vmean_update_cuda(vmean, g, 0.999)
    torch.cuda.synchronize()
    assert torch.isfinite(vmean).all()
    torch.testing.assert_close(vmean.cpu(), torch.full((2, 1), 300.0 ** 2 * (1 - 0.999)), rtol=1e-3, atol=0)


def test_bf16_vmean_is_the_model_dtype_square(dev):
    """bf16 grads square and average in bf16 (torch's own expression on the
    host), then the EMA runs in fp32: bit-identical."""
    from gefen.kernels.automatic_vmean import automatic_vmean_update_cuda
    gen = torch.Generator().manual_seed(0)
    g = (torch.randn(4, 16, generator=gen) * 3).to(torch.bfloat16)
    vmean = torch.rand(4, 1, generator=gen, dtype=torch.float32)
    expected = vmean.clone()
    expected.mul_(0.999).add_(torch.mean(g * g, dim=1, keepdim=True), alpha=1 - 0.999)
    out = vmean.to(dev)
    automatic_vmean_update_cuda(out, g.to(dev), 0.999)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), expected)


def _clone_tree(v):
    if torch.is_tensor(v):
        return v.detach().clone()
    if isinstance(v, dict):
        return {k: _clone_tree(x) for k, x in v.items()}
    if isinstance(v, (list, tuple)):
        return type(v)(_clone_tree(x) for x in v)
    return v


def _same_tree(a, b):
    if torch.is_tensor(b):
        return torch.is_tensor(a) and a.dtype == b.dtype and torch.equal(a.to_dense() if a.is_sparse else a,
                                                                          b.to_dense() if b.is_sparse else b)
    if isinstance(b, dict):
        return isinstance(a, dict) and set(a) == set(b) and all(_same_tree(a[k], b[k]) for k in b)
    if isinstance(b, (list, tuple)):
        return len(a) == len(b) and all(_same_tree(x, y) for x, y in zip(a, b))
    return a == b


@pytest.mark.parametrize("kind", ["gefen", "muon", "hybrid_gefen", "hybrid_adamw"])
def test_later_sparse_gradient_is_refused_before_any_mutation(dev, kind):
    """tests/test_step_preflight_atomicity.py (reference): once the first
    parameter has state, a step whose second gradient is sparse raises before
    anything moves: parameters, every state tensor, the global step and the
    codebook are unchanged."""
    from gefen import Gefen, GefenMuon, GefenMuonHybrid
    gen = torch.Generator().manual_seed(991)
    first = nn.Parameter((torch.randn(8, 8, generator=gen) * 0.02).to(dev))
    invalid = nn.Parameter(torch.eye(8, device=dev).to_sparse())
    if kind == "gefen":
        opt = Gefen([("first", first), ("invalid", invalid)], lr=2e-3, factored_v_2d=False)
    elif kind == "muon":
        opt = GefenMuon([("first", first), ("invalid", invalid)], lr=2e-3, ns_steps=1)
    else:
        opt = GefenMuonHybrid([("first", first)], [("invalid", invalid)], lr=2e-3, ns_steps=1,
                              ns_schedule="standard", normuon=False, backup_optimizer=kind.split("_")[1])
    first.grad = torch.full_like(first, 0.002)
    opt.step()
    opt.zero_grad(set_to_none=True)
    first.grad = torch.full_like(first, -0.003)
    invalid.grad = torch.eye(8, device=dev).to_sparse()
    torch.cuda.synchronize()
    children = [c for c in ((opt.muon, opt.backup) if kind.startswith("hybrid") else (opt,)) if isinstance(c, Gefen)]
    before = (first.detach().clone(), _clone_tree(opt.state_dict()),
              [(c._gefen_global_step, _clone_tree(c._gefen_codebook)) for c in children])
    with pytest.raises(RuntimeError, match="sparse|strided|layout"):
        opt.step()
    torch.cuda.synchronize()
    assert torch.equal(first, before[0])
    assert _same_tree(opt.state_dict(), before[1])
    for c, (gs, cb) in zip(children, before[2]):
        assert c._gefen_global_step == gs and _same_tree(c._gefen_codebook, cb)
