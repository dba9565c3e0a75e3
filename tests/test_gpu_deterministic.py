"""deterministic=True (gefen.py:1048-1057; reference tests/test_deterministic_mode.py):
the same inputs give bit-identical results run after run.

Every sum of the step runs in a fixed order here: the factored row / column
sums go through float64 per-tile partials, and the block path's per-block
sums of squares through a fixed-order segmented reduction with per-workgroup
records (no float atomics; block maxima use integer atomic max, exact in any
order).  With deterministic=True, block-path transposed views take the
contiguous route (the view kernels accumulate with atomics).  This test runs
a mixed set twice, in fresh optimizers, and compares every state tensor and
parameter bit for bit after every step (tests/det_workload.py); the block
sums cover blocks that span many stats workgroups, several blocks per wave,
and the one-element-per-item kernel (P % 8 != 0).  The same workload runs in
two child processes as well, and a grad view at an element offset (not
16-byte aligned) must step like an aligned one.
"""
import os
import subprocess
import sys
import tempfile

import numpy as np
import pytest
import torch

import det_workload

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


@pytest.mark.parametrize("factored", [True, False])
def test_deterministic_runs_are_bit_identical(dev, factored):
    print("deterministic repeat factored=%s" % factored, flush=True)
    a = det_workload.run(dev, factored)
    b = det_workload.run(dev, factored)
    for s, (sa, sb) in enumerate(zip(a, b)):
        for name in sa:
            for k in sa[name]:
                assert torch.equal(sa[name][k], sb[name][k]), (s, name, k)


@pytest.mark.parametrize("factored", [True, False])
def test_two_processes_are_bit_identical(dev, factored):
    """Reference tests/test_deterministic_mode.py:433-441 (replicas end
    bit-identical): the same workload in two fresh processes, one after the
    other on the one GPU (so nothing process-dependent -- plan caches,
    allocation addresses -- can feed an order), and in this process; every
    state tensor and parameter after every step compared bit for bit."""
    mode = "factored" if factored else "block"
    here = det_workload.run(dev, factored)
    outs = []
    with tempfile.TemporaryDirectory() as d:
        for i in range(2):
            out = os.path.join(d, "run%d.npz" % i)
            print("deterministic child %d (%s)" % (i, mode), flush=True)
            res = subprocess.run([sys.executable, os.path.join(HERE, "det_workload.py"), out, mode],
                                 capture_output=True, text=True, timeout=240)
            assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-4000:]
            with np.load(out) as z:
                outs.append({k: z[k].copy() for k in z.files})
    a, b = outs
    assert set(a) == set(b) and a
    for k in a:
        assert np.array_equal(a[k], b[k]), ("child runs differ", k)
    for s, snap in enumerate(here):
        for name, kv in snap.items():
            for k, v in kv.items():
                assert np.array_equal(a["s%d/%s/%s" % (s, name, k)], v.cpu().numpy()), ("parent differs", s, name, k)


@pytest.mark.parametrize("deterministic", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_block_sums_do_not_depend_on_grad_alignment(dev, deterministic, dtype):
    """The block path's per-block sums run in an order fixed by the shape:
    a grad that is a view at an element offset into a flat bucket (not
    16-byte aligned) steps bit-identically to an aligned copy -- vmean,
    indices, magnitudes and parameters."""
    from gefen import Gefen
    gen = torch.Generator().manual_seed(21)
    n, period = 1 << 20, 1 << 16
    init = (torch.randn(n, generator=gen) * 0.02).to(dtype)
    runs = []
    for offset in (0, 1):
        p = torch.nn.Parameter(init.clone().to(dev))
        opt = Gefen([("w", p)], lr=1e-3, weight_decay=0.01, deterministic=deterministic)
        opt.state[p]["automatic_period"] = period
        cb = np.load(os.path.join(HERE, "golden", "learn.npz"))["cb"]
        opt._gefen_codebook = torch.from_numpy(cb).float().to(dev)
        bucket = torch.empty(n + 8, dtype=dtype, device=dev)
        ggen = torch.Generator().manual_seed(22)
        for s in range(3):
            g = (torch.randn(n, generator=ggen) * 1e-3).to(dtype)
            view = bucket[offset:offset + n]
            view.copy_(g.to(dev))
            assert (view.data_ptr() % 16 == 0) == (offset == 0)
            p.grad = view
            opt.step()
        torch.cuda.synchronize()
        st = opt.state[p]
        runs.append({k: det_workload._bits(st[k]) for k in ("m_codebook", "m_magnitude", "vmean")})
        runs[-1]["p"] = det_workload._bits(p)
    for k in runs[0]:
        assert torch.equal(runs[0][k], runs[1][k]), (dtype, deterministic, k)
