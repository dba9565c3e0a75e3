"""The reference's kernel-wrapper names that gefen.py imports (gefen.py:28-51,
444-446) and that its tests call through `_load_extension()`, on the GPU:

  * `_load_extension()` objects carry the reference binding's function names
    (kernels/automatic_gefen_fused_binding.cpp:122-256, the vmean and
    histogram bindings);
  * gefen_factored_v_ema_cuda: the reference's own sweep
    (tests/test_factored_v_ema_parity.py:34-70: 60 random shapes, magnitudes
    1e-30 .. 1e10) bit-equal to the GPU aten chain it reproduces and to
    oracle.factored_v_ema;
  * automatic_vmean_update_cuda against oracle.vmean_update (1e-6 relative,
    float64 sums in another order);
  * gefen_exact_histogram_cuda against oracle.exact_histogram (exact counts);
  * automatic_gefen_fused_update_cuda (the legacy partial update) against
    oracle.partial_update: indices and magnitudes bit-exact, p within one ulp;
    lr = 0 leaves p untouched;
  * the binding-order entry points (`lut` positional) give the wrapper
    functions' results bit for bit, and reject a malformed LUT.
"""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import assert_within_ulp

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TDT = {orc.F32: torch.float32, orc.F16: torch.float16, orc.BF16: torch.bfloat16}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _cb():
    return np.load(os.path.join(GOLD, "learn.npz"))["cb"].astype(np.float32)


def test_extension_objects_carry_the_reference_names(dev):
    from gefen.kernels import automatic_gefen_fused, automatic_vmean, exact_histogram_fused
    ext = automatic_gefen_fused._load_extension()
    for name in ("automatic_gefen_fused_update_cuda", "automatic_gefen_fused_update_v2_cuda",
                 "automatic_gefen_fused_full_update_cuda", "automatic_gefen_fused_update_v2_full_cuda",
                 "gefen_quantized_momentum_update_cuda", "gefen_factored_update_cuda", "gefen_factored_v_ema_cuda"):
        assert callable(getattr(ext, name)), name
    assert callable(automatic_vmean._load_extension().automatic_vmean_update_cuda)
    assert callable(exact_histogram_fused._load_extension().gefen_exact_histogram_cuda)
    for name in ("automatic_vmean_update_cuda",):
        assert callable(getattr(automatic_vmean, name))
    assert callable(exact_histogram_fused.gefen_exact_histogram_cuda)
    assert callable(automatic_gefen_fused.automatic_gefen_fused_update_cuda)


def test_factored_v_ema_reference_sweep(dev):
    from gefen.kernels.automatic_gefen_fused import _load_extension
    mod = _load_extension()
    torch.manual_seed(0)
    total = 0
    for it in range(60):
        rows = int(torch.randint(1, 5000, (1,)).item())
        cols = int(torch.randint(1, 5000, (1,)).item())
        beta2 = float(torch.rand(()) * 0.2 + 0.8)
        scale_r = torch.logspace(-30, 10, rows, device=dev)
        scale_c = torch.logspace(-30, 10, cols, device=dev)
        v_row = (torch.randn(rows, device=dev) * scale_r).abs()
        v_col = (torch.randn(cols, device=dev) * scale_c).abs()
        row_sq = (torch.randn(rows, device=dev) * scale_r).square()
        col_sq = (torch.randn(cols, device=dev) * scale_c).square()
        ref_r = v_row.clone().mul_(beta2).add_(row_sq.clone().div_(float(cols)), alpha=1 - beta2)
        ref_c = v_col.clone().mul_(beta2).add_(col_sq.clone().div_(float(rows)), alpha=1 - beta2)
        got_r, got_c = v_row.clone(), v_col.clone()
        mod.gefen_factored_v_ema_cuda(got_r, got_c, row_sq, col_sq, beta2)
        torch.cuda.synchronize()
        tag = "sweep %d rows=%d cols=%d beta2=%r" % (it, rows, cols, beta2)
        assert torch.equal(got_r, ref_r), tag + " v_row vs aten chain"
        assert torch.equal(got_c, ref_c), tag + " v_col vs aten chain"
        o_r = orc.factored_v_ema(v_row.cpu().numpy(), row_sq.cpu().numpy(), cols, beta2)
        o_c = orc.factored_v_ema(v_col.cpu().numpy(), col_sq.cpu().numpy(), rows, beta2)
        np.testing.assert_array_equal(got_r.cpu().numpy(), o_r, err_msg=tag + " v_row vs oracle")
        np.testing.assert_array_equal(got_c.cpu().numpy(), o_c, err_msg=tag + " v_col vs oracle")
        total += rows + cols
    assert total > 100_000
    with pytest.raises(ValueError):
        mod.gefen_factored_v_ema_cuda(torch.zeros(3, device=dev), torch.zeros(0, device=dev),
                                      torch.zeros(3, device=dev), torch.zeros(0, device=dev), 0.9)


@pytest.mark.parametrize("dtype,n,period", [(orc.BF16, 4096, 512), (orc.F32, 3000, 24), (orc.F16, 999, 27),
                                            (orc.BF16, 1 << 20, 1 << 18)])
def test_vmean_update_matches_oracle(dev, dtype, n, period):
    from gefen.kernels.automatic_vmean import automatic_vmean_update_cuda
    rng = np.random.default_rng(n)
    v = np.abs(rng.standard_normal(n // period) * 1e-6).astype(np.float32)
    vmean = torch.from_numpy(v.copy()).view(-1, 1).to(dev)
    for step in range(3):
        g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(TDT[dtype])
        automatic_vmean_update_cuda(vmean, g.to(dev).view(-1, period), 0.999)
        torch.cuda.synchronize()
        v = orc.vmean_update(v, g.float().numpy(), period, dtype, 0.999)
        np.testing.assert_allclose(vmean.cpu().numpy().reshape(-1), v, rtol=1e-6, err_msg="step %d" % step)
        v = vmean.cpu().numpy().reshape(-1)


@pytest.mark.parametrize("dtype,n,period,bins", [(orc.BF16, 1 << 16, 256, 4096), (orc.F32, 29995, 7, 4096),
                                                 (orc.F16, 4096, 4096, 1024), (orc.BF16, 12288, 3, 37),
                                                 (orc.F32, 20000, 100, 100)])
def test_exact_histogram_matches_oracle(dev, dtype, n, period, bins):
    """Power-of-two bins: the torch path's binning, which the golden
    codebooks pin; other bin counts: the reference kernel's multiply by
    bins / 2 (the two forms agree for powers of two)."""
    from gefen.kernels.exact_histogram_fused import gefen_exact_histogram_cuda
    rng = np.random.default_rng(period)
    g = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    g[:period] = 0.0  # a block whose maximum is zero
    gt = torch.from_numpy(g).to(TDT[dtype])
    counts = torch.zeros(bins, dtype=torch.int64, device=dev)
    gefen_exact_histogram_cuda(gt.to(dev), period, counts)
    gefen_exact_histogram_cuda(gt.to(dev), period, counts)  # accumulates
    torch.cuda.synchronize()
    ref = orc.exact_histogram(gt.float().numpy(), period, bins, kernel_scale=bins & (bins - 1) != 0)
    np.testing.assert_array_equal(counts.cpu().numpy(), 2 * ref)
    with pytest.raises(ValueError):
        gefen_exact_histogram_cuda(gt.to(dev), period, torch.zeros(bins, dtype=torch.int32, device=dev))
    with pytest.raises(ValueError):
        gefen_exact_histogram_cuda(gt.to(dev), period, torch.zeros(4097, dtype=torch.int64, device=dev))


@pytest.mark.parametrize("dtype,n,period,use_v2", [(orc.BF16, 4096, 64, None), (orc.F32, 3000, 24, True),
                                                   (orc.F16, 999, 27, False), (orc.BF16, 1 << 20, 1 << 18, None)])
def test_partial_update_matches_oracle(dev, dtype, n, period, use_v2):
    from gefen.kernels.automatic_gefen_fused import automatic_gefen_fused_update_cuda
    rng = np.random.default_rng(n + period)
    cb = _cb()
    cb_dev = torch.from_numpy(cb).to(dev)
    nb = n // period
    p0 = torch.from_numpy((rng.standard_normal(n) * 0.02).astype(np.float32)).to(TDT[dtype])
    p = p0.to(dev)
    idx = torch.zeros(nb, period, dtype=torch.uint8, device=dev)
    mag = torch.zeros(nb, 1, dtype=torch.float32, device=dev)
    ref = {"p": p0.float().numpy(), "idx": np.zeros(n, np.uint8), "mag": np.zeros(nb, np.float32)}
    for step in range(3):
        g = torch.from_numpy((rng.standard_normal(n) * 1e-3).astype(np.float32)).to(TDT[dtype])
        stepsize = (rng.uniform(0.5, 2.0, nb) * 100).astype(np.float32)
        lr = 0.0 if step == 1 else 6e-5
        automatic_gefen_fused_update_cuda(p, g.to(dev).view(nb, period), idx, mag,
                                          torch.from_numpy(stepsize).view(-1, 1).to(dev), cb_dev, False, 0.9, lr,
                                          use_v2=use_v2)
        torch.cuda.synchronize()
        p1, i1, m1 = orc.partial_update(ref["p"], g.float().numpy(), ref["idx"], ref["mag"], stepsize, period, cb,
                                        dtype, beta1=0.9, lr=lr)
        tag = "step %d lr %g" % (step, lr)
        np.testing.assert_array_equal(idx.cpu().numpy().reshape(-1), i1, err_msg=tag)
        np.testing.assert_array_equal(mag.cpu().numpy().reshape(-1), m1, err_msg=tag)
        got = p.float().cpu().numpy()
        if lr == 0.0:
            np.testing.assert_array_equal(got, ref["p"], err_msg=tag + " p untouched")
        assert_within_ulp(got, p1, dtype, tag + " p", atol=1e-6 * 6e-5)
        ref = {"p": got, "idx": i1, "mag": m1}


def test_binding_order_entry_points_match_wrappers(dev):
    """`_load_extension().gefen_factored_update_cuda(..., codebook, lut, cols, ...)`
    and the full / momentum entries give the wrapper functions' results."""
    from gefen.kernels import automatic_gefen_fused as fused
    ext = fused._load_extension()
    rng = np.random.default_rng(5)
    cb_dev = torch.from_numpy(_cb()).to(dev)
    lut = fused._codebook_search_lut(cb_dev)
    rows, cols, period = 64, 96, 768
    nb = rows * cols // period

    def fresh():
        return {"p": torch.from_numpy((rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)).to(dev),
                "idx": torch.zeros(nb, period, dtype=torch.uint8, device=dev),
                "mag": torch.zeros(nb, 1, device=dev), "vr": torch.zeros(rows, device=dev),
                "vc": torch.zeros(cols, device=dev), "vm": torch.zeros(nb, 1, device=dev)}

    g = torch.from_numpy((rng.standard_normal((rows, cols)) * 1e-3).astype(np.float32)).to(dev)
    a, b = fresh(), None
    b = {k: v.clone() for k, v in a.items()}
    args = (0.9, 0.999, 6e-5, 1e-8, 1.0 / (1 - 0.999), 1.0 / (1 - 0.9), 1 - 6e-7)
    fused.gefen_factored_update_cuda(a["p"], g.view(nb, period), a["idx"], a["mag"], a["vr"], a["vc"], cb_dev, cols,
                                     *args)
    ext.gefen_factored_update_cuda(b["p"], g.view(nb, period), b["idx"], b["mag"], b["vr"], b["vc"], cb_dev, lut,
                                   cols, *args)
    a2, b2 = fresh(), None
    b2 = {k: v.clone() for k, v in a2.items()}
    fused.automatic_gefen_fused_full_update_cuda(a2["p"].view(-1), g.view(nb, period), a2["idx"], a2["mag"],
                                                 a2["vm"], cb_dev, False, *args)
    ext.automatic_gefen_fused_update_v2_full_cuda(b2["p"].view(-1), g.view(nb, period), b2["idx"], b2["mag"],
                                                  b2["vm"], cb_dev, lut, False, *args)
    mo_a = torch.empty(rows * cols, device=dev)
    mo_b = torch.empty(rows * cols, device=dev)
    ia, ma = a2["idx"].clone(), a2["mag"].clone()
    ib, mb = ia.clone(), ma.clone()
    fused.gefen_quantized_momentum_update_cuda(g.view(nb, period), ia, ma, cb_dev, mo_a, 0.95, nesterov=True)
    ext.gefen_quantized_momentum_update_cuda(g.view(nb, period), ib, mb, cb_dev, lut, mo_b, 0.95, False, 0, None,
                                             True)
    torch.cuda.synchronize()
    for x, y in ((a, b), (a2, b2)):
        for k in x:
            assert torch.equal(x[k], y[k]), k
    assert torch.equal(mo_a, mo_b) and torch.equal(ia, ib) and torch.equal(ma, mb)
    with pytest.raises(ValueError):
        ext.gefen_factored_update_cuda(b["p"], g.view(nb, period), b["idx"], b["mag"], b["vr"], b["vc"], cb_dev,
                                       lut.to(torch.int32), cols, *args)


def test_grad_histogram_dump_hook(dev, tmp_path, monkeypatch):
    """gefen.py:3095-3150: with LIST_STEPS_SAVE_HIST_GRAD = [1] the step at
    global step 1 writes <prefix>_grad_hist_step_1.pt whose counts are the
    block-normalised histogram of that step's grads (oracle.exact_histogram,
    4096 bins, each tensor at its period); capturable=True refuses."""
    from gefen import Gefen, quantization
    monkeypatch.setattr(quantization, "LIST_STEPS_SAVE_HIST_GRAD", [1])
    monkeypatch.setattr(quantization, "SAVE_CODEBOOK_PREFIX", str(tmp_path / "dump" / "cb"))
    gen = torch.Generator().manual_seed(8)
    w = torch.nn.Parameter((torch.randn(64, 96, generator=gen) * 0.02).to(torch.bfloat16).to(dev))
    b = torch.nn.Parameter((torch.randn(96, generator=gen) * 0.02).to(torch.bfloat16).to(dev))
    opt = Gefen([("w", w), ("b", b)], lr=1e-3)
    grads = []
    for s in range(3):
        gw = (torch.randn(64, 96, generator=gen) * 1e-3).to(torch.bfloat16)
        gb = (torch.randn(96, generator=gen) * 1e-2).to(torch.bfloat16)
        grads.append((gw, gb))
        w.grad, b.grad = gw.to(dev), gb.to(dev)
        opt.step()
    torch.cuda.synchronize()
    files = sorted(os.listdir(tmp_path / "dump"))
    assert files == ["cb_grad_hist_step_1.pt"], files
    d = torch.load(tmp_path / "dump" / files[0], weights_only=True)
    gw, gb = grads[1]
    ref = orc.exact_histogram(gw.float().numpy(), opt.state[w]["automatic_period"], 4096)
    orc.exact_histogram(gb.float().numpy(), opt.state[b]["automatic_period"], 4096, counts=ref)
    np.testing.assert_array_equal(d["hist"].numpy(), ref.astype(np.float32))
    assert d["num_samples"] == w.numel() + b.numel() and d["num_bins"] == 4096
    opt_c = Gefen([("w2", torch.nn.Parameter(w.detach().clone()))], lr=1e-3, capturable=True)
    list(opt_c.param_groups[0]["params"])[0].grad = gw.to(dev)
    monkeypatch.setattr(quantization, "LIST_STEPS_SAVE_HIST_GRAD", [0])
    with pytest.raises(ValueError, match="capturable"):
        opt_c.step()
