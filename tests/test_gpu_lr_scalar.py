"""A device (tensor) lr on MI355X, as the reference pins it
(tests/test_lr_item_no_sync.py there): after warm-up a constant tensor lr
adds no Tensor.item() host syncs over a python-float lr, in Gefen and in
GefenMuon; a constant tensor lr, an in-place scheduled one and a fresh tensor
per step all give the float lr's trajectory bit for bit."""
import pytest
import torch

pytestmark = pytest.mark.gpu

SPEC = [(256, 256), (384, 256), (256, 384), (512, 256), (256, 512)]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


class _ItemCount:
    def __enter__(self):
        self.n = 0
        self._orig = torch.Tensor.item

        def counted(t):
            self.n += 1
            return self._orig(t)
        torch.Tensor.item = counted
        return self

    def __exit__(self, *exc):
        torch.Tensor.item = self._orig


def _build(kind, lr, dev):
    from gefen import Gefen, GefenMuon
    gen = torch.Generator(device=dev).manual_seed(1234)
    ps = [("layers.%d.weight" % i, torch.nn.Parameter(torch.randn(r, c, device=dev, generator=gen).to(torch.bfloat16)
                                                         * 0.02)) for i, (r, c) in enumerate(SPEC)]
    if kind == "muon":
        return GefenMuon(ps, lr=lr, ns_steps=2), [p for _, p in ps]
    return Gefen(ps, lr=lr, weight_decay=0.01), [p for _, p in ps]


def _run(opt, params, dev, steps, schedule=None):
    gen = torch.Generator(device=dev).manual_seed(99)
    for s in range(steps):
        for p in params:
            p.grad = (torch.randn(p.shape, device=dev, generator=gen) * 1e-3).to(torch.bfloat16)
        if schedule is not None:
            schedule(opt, s)
        opt.step()
    torch.cuda.synchronize()


@pytest.mark.parametrize("kind", ["gefen", "muon"])
def test_constant_tensor_lr_adds_no_item_syncs(dev, kind):
    counts = []
    for lr in (1e-3, torch.tensor(1e-3, device=dev)):
        opt, ps = _build(kind, lr, dev)
        _run(opt, ps, dev, 3)
        with _ItemCount() as c:
            _run(opt, ps, dev, 5)
        counts.append(c.n)
    assert counts[1] == counts[0], counts


@pytest.mark.parametrize("kind", ["gefen", "muon"])
def test_tensor_lr_trajectories_are_the_float_ones(dev, kind):
    lr0 = float(torch.tensor(1e-3))  # the fp32 value a tensor lr holds
    base = [lr0 * (0.5 ** s) for s in range(4)]  # halving is exact in fp32

    def run(make_lr, sched):
        opt, ps = _build(kind, make_lr(), dev)
        _run(opt, ps, dev, 4, sched)
        return [p.detach().clone() for p in ps]

    def float_sched(opt, s):
        opt.param_groups[0]["lr"] = base[s]

    def inplace_sched(opt, s):
        if s:
            opt.param_groups[0]["lr"].mul_(0.5)

    def fresh_sched(opt, s):
        opt.param_groups[0]["lr"] = torch.tensor(base[s], device=dev)

    ref = run(lambda: lr0, float_sched)
    for sched in (inplace_sched, fresh_sched):
        got = run(lambda: torch.tensor(1e-3, device=dev), sched)
        for a, b in zip(ref, got):
            assert torch.equal(a, b), sched.__name__
    const = run(lambda: torch.tensor(1e-3, device=dev), None)
    assert any(not torch.equal(a, b) for a, b in zip(ref, const))
