"""deterministic=True (gefen.py:1048-1057; reference tests/test_deterministic_mode.py):
the same inputs give bit-identical results run after run.

Every sum of the step runs in a fixed order here: the factored row / column
sums go through float64 per-tile partials, and the block path's per-block
sums of squares through a fixed-order segmented reduction with per-workgroup
records (no float atomics; block maxima use integer atomic max, exact in any
order).  With deterministic=True, block-path transposed views take the
contiguous route (the view kernels accumulate with atomics).  This test runs
a mixed set twice, in fresh optimizers, and compares every state tensor and
parameter bit for bit after every step; the block sums cover blocks that span
many stats workgroups, several blocks per wave, and the one-element-per-item
kernel (P % 8 != 0).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SPECS = [("w2d", (96, 128)), ("big1d", (1 << 21,)), ("odd1d", (99999,)), ("fine1d", (122880,)),
         ("wT", (64, 96))]
PERIODS = {"big1d": 1 << 19, "odd1d": 11111, "fine1d": 40, "w2d": 768, "wT": 768}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _bits(t):
    """The tensor's bytes in logical order (a bitwise snapshot)."""
    return t.detach().contiguous().clone().reshape(-1).view(torch.uint8)


def _run(dev, factored):
    from gefen import Gefen
    gen = torch.Generator().manual_seed(4)
    params = []
    for name, shape in SPECS:
        data = (torch.randn(*shape, generator=gen) * 0.02).to(torch.bfloat16)
        if name == "wT":
            p = torch.nn.Parameter(data.t().contiguous().to(dev).t())
        else:
            p = torch.nn.Parameter(data.to(dev))
        params.append((name, p))
    opt = Gefen(params, lr=1e-3, betas=(0.9, 0.999), weight_decay=0.01, factored_v_2d=factored,
                deterministic=True)
    for name, p in params:
        opt.state[p]["automatic_period"] = PERIODS[name]
    cb = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "learn.npz"))["cb"]
    opt._gefen_codebook = torch.from_numpy(cb).float().to(dev)
    snaps = []
    for s in range(4):
        for name, p in params:
            g = (torch.randn(*p.shape, generator=gen) * 10 ** (-3 + s % 2)).to(torch.bfloat16)
            p.grad = g.t().contiguous().to(dev).t() if name == "wT" else g.to(dev)
        opt.step()
        torch.cuda.synchronize()
        snap = {}
        for name, p in params:
            st = opt.state[p]
            snap[name] = {k: _bits(v) for k, v in st.items() if torch.is_tensor(v) and not k.startswith("_")}
            snap[name]["p"] = _bits(p)
        snaps.append(snap)
    return snaps


@pytest.mark.parametrize("factored", [True, False])
def test_deterministic_runs_are_bit_identical(dev, factored):
    print("deterministic repeat factored=%s" % factored, flush=True)
    a = _run(dev, factored)
    b = _run(dev, factored)
    for s, (sa, sb) in enumerate(zip(a, b)):
        for name in sa:
            for k in sa[name]:
                assert torch.equal(sa[name][k], sb[name][k]), (s, name, k)
