"""Step-1 kernels on the GPU against the oracle and the reference's goldens:
the block-absmax histogram (integer counts: exact), the period-search errors
(float64: 1e-12 relative) and the chosen period, and the whole first optimizer
step of the Gefen class (period, learned codebook, then parity of the state)."""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import assert_within_ulp

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _hist_gpu(g_dev, period, bins=4096):
    from gefen.kernels import _native
    from gefen.kernels.automatic_gefen_fused import _dtype_code, _stream
    counts = torch.zeros(bins, dtype=torch.int64, device=g_dev.device)
    flat = g_dev.reshape(-1).contiguous()
    _native.check(_native.load().gefenx_exact_histogram(
        flat.data_ptr(), _dtype_code(flat.dtype), flat.numel(), period, counts.data_ptr(), bins,
        _stream(flat.device)))
    return counts.cpu().numpy()


@pytest.mark.parametrize("n,period,dt", [(4096, 64, torch.bfloat16), (1 << 20, 1 << 19, torch.float32),
                                         (300006, 7, torch.float16), (5000, 5000, torch.bfloat16),
                                         (200000, 100000, torch.bfloat16)])
def test_histogram_counts_exact(dev, n, period, dt):
    gen = torch.Generator().manual_seed(n + period)
    g = (torch.randn(n, generator=gen) * 1e-3).to(dt)
    g[: min(64, n)] = 0  # an all-zero prefix (zero absmax when the block is that small)
    got = _hist_gpu(g.to(dev), period)
    ref = orc.exact_histogram(g.float().numpy(), period)
    np.testing.assert_array_equal(got, ref)
    print("case hist", n, period, dt, flush=True)


def test_learned_codebook_matches_reference_golden(dev):
    from gefen.kernels import _native
    z = np.load(os.path.join(GOLD, "learn.npz"))
    counts = np.zeros(4096, np.int64)
    for tag in ("w", "b"):
        g = torch.from_numpy(z["g_" + tag]).to(dev)
        counts += _hist_gpu(g, int(z["period_" + tag]))
    centers, cnts = orc.histogram_stats(counts)
    from gefen import quantization
    stats = {"active_centers": torch.from_numpy(centers), "active_counts": torch.from_numpy(cnts)}
    cb = quantization.exact_dp(stats, 256, True).numpy()
    np.testing.assert_array_equal(cb, z["cb"])
    _native.load()


def test_device_exact_dp_matches_host_and_golden(dev):
    """gefenx_exact_dp_device (DP levels on the GPU) against the reference's
    learned codebook and, bit for bit, against the host solver on random
    histograms: all active bins, sparse bins, fewer bins than centres, k
    below 256, and ties (equal counts on a symmetric grid)."""
    from gefen import quantization
    z = np.load(os.path.join(GOLD, "learn.npz"))
    counts = np.zeros(4096, np.int64)
    for tag in ("w", "b"):
        counts += _hist_gpu(torch.from_numpy(z["g_" + tag]).to(dev), int(z["period_" + tag]))
    centers, cnts = orc.histogram_stats(counts)
    stats = {"active_centers": torch.from_numpy(centers), "active_counts": torch.from_numpy(cnts)}
    np.testing.assert_array_equal(quantization.exact_dp(stats, 256, True, device=dev).numpy(), z["cb"])
    rng = np.random.default_rng(7)
    grid = (np.arange(4096, dtype=np.float32) + 0.5) / 2048 - 1
    cases = [(4096, 256, True), (700, 256, True), (100, 256, True), (300, 16, True), (513, 64, False)]
    for n, k, force in cases:
        sel = np.sort(rng.choice(4096, size=n, replace=False))
        c = grid[sel].astype(np.float32)
        w = np.floor(rng.pareto(1.2, size=n) * 50 + 1).astype(np.float32)
        st = {"active_centers": torch.from_numpy(c), "active_counts": torch.from_numpy(w)}
        host = quantization.exact_dp(st, k, force).numpy()
        devr = quantization.exact_dp(st, k, force, device=dev).numpy()
        np.testing.assert_array_equal(devr, host, err_msg="n=%d k=%d force=%s" % (n, k, force))
    st = {"active_centers": torch.from_numpy(grid[::8].copy()),
          "active_counts": torch.ones(512, dtype=torch.float32)}
    np.testing.assert_array_equal(quantization.exact_dp(st, 256, True, device=dev).numpy(),
                                  quantization.exact_dp(st, 256, True).numpy(), err_msg="ties")


def test_period_search_matches_reference_golden(dev):
    from gefen import partitioning
    z = np.load(os.path.join(GOLD, "period.npz"))
    for tag in sorted(k[2:] for k in z.files if k.startswith("g_")):
        g = torch.from_numpy(z["g_" + tag]).to(dev)
        errs = partitioning.block_variance_errors_device(g, partitioning.divisors(g.numel()))
        np.testing.assert_allclose(errs, z["errs_" + tag], rtol=1e-12, atol=1e-300)
        period = partitioning.find_period_by_block_variance(
            g.reshape(-1), print_results=False, parameter_shape=tuple(g.shape), backend="cuda_kernel",
            input_is_squared=False)
        assert period == int(z["period_" + tag]), tag
        print("case period", tag, period, flush=True)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_period_errors_large_blocks(dev, dt):
    gen = torch.Generator().manual_seed(3)
    g = (torch.randn(8, 65536 * 3, generator=gen) * 1e-3).to(dt)
    divs = [65536 * 3, 65536 * 6, 65536 * 12, 4096, 3 * 8192]
    from gefen import partitioning
    got = partitioning.block_variance_errors_device(g.to(dev), divs)
    vals = (g.float().numpy().reshape(-1) ** 2).astype(np.float32).astype(np.float64)
    ref = [orc.block_variance_error(vals, d) for d in divs]
    np.testing.assert_allclose(got, ref, rtol=1e-10)


def test_gefen_class_first_steps_match_oracle(dev):
    """Gefen.step on the GPU: periods from the search, the learned codebook
    and three steps of state against the oracle run on the same inputs."""
    from gefen import Gefen
    gen = torch.Generator().manual_seed(11)
    shapes = {"w": (96, 128), "b": (128,), "e": (64, 48)}
    init = {k: (torch.randn(*s, generator=gen) * 0.02).to(torch.bfloat16) for k, s in shapes.items()}
    params = [(k, torch.nn.Parameter(v.clone().to(dev))) for k, v in init.items()]
    opt = Gefen(params, lr=6e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    ref = {k: {"p": v.float().numpy()} for k, v in init.items()}
    cb = None
    for s in range(1, 4):
        grads = {k: (torch.randn(*shp, generator=gen) * 1e-3).to(torch.bfloat16) for k, shp in shapes.items()}
        for name, p in params:
            p.grad = grads[name].to(dev)
        opt.step()
        torch.cuda.synchronize()
        if s == 1:
            for name, p in params:
                g = grads[name].float().numpy()
                per = orc.resolve_period(g, g.shape)
                assert opt.state[p]["automatic_period"] == per, name
                ref[name]["period"] = per
            cb = orc.learn_codebook([(grads[n].float().numpy(), ref[n]["period"]) for n in shapes])
            np.testing.assert_array_equal(opt._gefen_codebook.cpu().numpy(), cb)
        for name, p in params:
            r = ref[name]
            g = grads[name].float().numpy()
            per = r["period"]
            n = g.size
            if "idx" not in r:
                r["idx"] = np.zeros(n, np.uint8)
                r["mag"] = np.zeros(n // per, np.float32)
                if g.ndim == 2:
                    r["v_row"] = np.zeros(g.shape[0], np.float32)
                    r["v_col"] = np.zeros(g.shape[1], np.float32)
                else:
                    r["vmean"] = np.zeros(n // per, np.float32)
            kw = dict(beta1=0.9, beta2=0.999, lr=6e-5, eps=1e-8, bc1=1 - 0.9 ** s, bc2=1 - 0.999 ** s, wd=0.01)
            if g.ndim == 2:
                r["p"], r["idx"], r["mag"], r["v_row"], r["v_col"] = orc.factored_step(
                    r["p"], g, r["idx"], r["mag"], r["v_row"], r["v_col"], per, cb, orc.BF16, **kw)
            else:
                r["p"], r["idx"], r["mag"], r["vmean"] = orc.block_step(
                    r["p"], g, r["idx"], r["mag"], r["vmean"], per, cb, orc.BF16, **kw)
            st = opt.state[p]
            np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), r["idx"])
            np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), r["mag"])
            assert_within_ulp(p.detach().float().cpu().numpy(), r["p"], orc.BF16, "step1 p", atol=1e-6 * kw["lr"])
            # keep the oracle on the GPU's sums (summation order differs at 1e-7)
            r["p"] = p.detach().float().cpu().numpy()
            if g.ndim == 2:
                np.testing.assert_allclose(st["v_row"].cpu().numpy(), r["v_row"], rtol=1e-6)
                r["v_row"], r["v_col"] = st["v_row"].cpu().numpy(), st["v_col"].cpu().numpy()
            else:
                np.testing.assert_allclose(st["vmean"].cpu().numpy().reshape(-1), r["vmean"], rtol=1e-6)
                r["vmean"] = st["vmean"].cpu().numpy().reshape(-1)
        print("case gefen-class step", s, "ok", flush=True)
