"""BASELINE configs[0] on the GPU: the reference's own 10-step trajectory of a
4096x4096 fp32 weight plus a 4096 fp32 bias (tests/golden/config1.npz, written
by the reference's CPU step), replayed through this build's `Gefen` class.

Step 1 runs the GPU period search and codebook learning; both must give the
reference's period and codebook exactly.  Then, every step:
  - the sha256 of the whole 16,777,216-entry index array of the weight and
    the full index array of the bias: bit-exact;
  - magnitudes: bit-exact;
  - v_row / v_col / vmean: within 1e-6 relative (float64 sums in another
    order than torch's CPU cascade);
  - the weight subsample (every 4099th element) and the whole bias: within
    1e-6 of max(|p0|, |p|) per element (a last-bit skew of the stepsize flips
    a rounding of p, and that ulp, taken while |p| was near |p0|, is carried
    along where p later shrinks; the oracle's own free run stays within 2 ulps
    of that scale).
"""
import hashlib
import os
import sys

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LR, BETAS, EPS, WD = 6e-5, (0.9, 0.999), 1e-8, 0.01
SUB = 4099


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _inputs(step=None):
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(4096, 4096, generator=gen) * 0.02
    b = torch.randn(4096, generator=gen) * 0.02
    if step is None:
        return w, b
    gt = torch.Generator().manual_seed(1000 + step)
    return torch.randn(4096, 4096, generator=gt) * 1e-3, torch.randn(4096, generator=gt) * 1e-3


def _assert_p_close(got, ref, p0, what):
    scale = np.maximum(np.abs(p0), np.abs(ref)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bad = err > 1e-6 * scale
    assert not bad.any(), "%s: %d elements beyond 1e-6 of max(|p0|,|p|), worst %.3g" % (
        what, int(bad.sum()), float((err / np.maximum(scale, 1e-38)).max()))


@pytest.mark.parametrize("multi_tensor", [True, False], ids=["multi", "single"])
def test_config1_trajectory_on_gpu(multi_tensor, monkeypatch):
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from gefen import Gefen
    monkeypatch.setenv("GEFENX_MULTI_TENSOR", "1" if multi_tensor else "0")
    dev = torch.device("cuda", 0)
    z = np.load(os.path.join(GOLD, "config1.npz"))
    w0, b0 = _inputs()
    w0_sub, b0_np = w0.reshape(-1)[::SUB].numpy().copy(), b0.numpy().copy()
    W = torch.nn.Parameter(w0.to(dev))
    B = torch.nn.Parameter(b0.to(dev))
    opt = Gefen([("weight", W), ("bias", B)], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD,
                factored_v_2d=True)
    for s in range(1, 11):
        gw, gb = _inputs(s)
        W.grad, B.grad = gw.to(dev), gb.to(dev)
        opt.step()
        torch.cuda.synchronize()
        sw, sb = opt.state[W], opt.state[B]
        tag = "step %d" % s
        print("config1 %s %s" % ("multi" if multi_tensor else "single", tag), flush=True)
        sys.stdout.flush()
        if s == 1:
            assert sw["automatic_period"] == int(z["period_weight"])
            assert sb["automatic_period"] == int(z["period_bias"])
            np.testing.assert_array_equal(opt._gefen_codebook.cpu().numpy(), z["codebook"])
        idx_w = sw["m_codebook"].cpu().numpy().reshape(-1)
        assert _sha(idx_w) == str(z["sha_idx%d_weight" % s]), tag + " weight indices (sha256)"
        np.testing.assert_array_equal(idx_w[::SUB], z["idx_sub%d_weight" % s], err_msg=tag)
        np.testing.assert_array_equal(sw["m_magnitude"].cpu().numpy().reshape(-1), z["mag%d_weight" % s],
                                      err_msg=tag + " weight magnitudes")
        np.testing.assert_allclose(sw["v_row"].cpu().numpy(), z["v_row%d_weight" % s], rtol=1e-6, atol=0,
                                   err_msg=tag + " v_row")
        np.testing.assert_allclose(sw["v_col"].cpu().numpy(), z["v_col%d_weight" % s], rtol=1e-6, atol=0,
                                   err_msg=tag + " v_col")
        _assert_p_close(W.detach().cpu().numpy().reshape(-1)[::SUB], z["p_sub%d_weight" % s], w0_sub,
                        tag + " weight")
        np.testing.assert_array_equal(sb["m_codebook"].cpu().numpy().reshape(-1), z["idx%d_bias" % s],
                                      err_msg=tag + " bias indices")
        np.testing.assert_array_equal(sb["m_magnitude"].cpu().numpy().reshape(-1), z["mag%d_bias" % s],
                                      err_msg=tag + " bias magnitudes")
        np.testing.assert_allclose(sb["vmean"].cpu().numpy().reshape(-1), z["vmean%d_bias" % s], rtol=1e-6,
                                   atol=0, err_msg=tag + " vmean")
        _assert_p_close(B.detach().cpu().numpy(), z["p%d_bias" % s], b0_np, tag + " bias")


def _oracle_trajectory(z):
    """The oracle's 10 steps of configs[0] from the golden period and
    codebook; each step's weight indices are checked against the golden
    sha256 (the reference's own), so every state here is the reference's."""
    from oracle import oracle as orc
    w0, b0 = _inputs()
    pw, pb = int(z["period_weight"]), int(z["period_bias"])
    cb = z["codebook"]
    st = {"W": w0.numpy().copy(), "B": b0.numpy().copy(),
          "iw": np.zeros(4096 * 4096, np.uint8), "mw": np.zeros(4096 * 4096 // pw, np.float32),
          "vr": np.zeros(4096, np.float32), "vc": np.zeros(4096, np.float32),
          "ib": np.zeros(4096, np.uint8), "mb": np.zeros(4096 // pb, np.float32), "vm": np.zeros(4096 // pb, np.float32)}
    states = [dict(st)]
    for s in range(1, 11):
        gw, gb = _inputs(s)
        bc1, bc2 = 1 - BETAS[0] ** s, 1 - BETAS[1] ** s
        kw = dict(beta1=BETAS[0], beta2=BETAS[1], lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=WD)
        W, iw, mw, vr, vc = orc.factored_step(st["W"], gw.numpy(), st["iw"], st["mw"], st["vr"], st["vc"], pw, cb,
                                              orc.F32, **kw)
        B, ib, mb, vm = orc.block_step(st["B"], gb.numpy(), st["ib"], st["mb"], st["vm"], pb, cb, orc.F32, **kw)
        assert _sha(iw) == str(z["sha_idx%d_weight" % s]), "oracle step %d weight indices (sha256)" % s
        np.testing.assert_array_equal(ib, z["idx%d_bias" % s])
        st = {"W": W, "B": B, "iw": iw, "mw": mw, "vr": vr, "vc": vc, "ib": ib, "mb": mb, "vm": vm}
        states.append(st)
    return states


def test_config1_each_step_from_the_reference_state():
    """Every step restarts from the reference's state of the step before
    (parameters, indices, magnitudes, v_row / v_col / vmean set on the GPU
    optimizer), so no earlier rounding is carried: indices and magnitudes
    bit-exact, v within 1e-6, and every weight and bias element within
    1e-6 * |p| of the reference's (fp32)."""
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from gefen import Gefen
    dev = torch.device("cuda", 0)
    z = np.load(os.path.join(GOLD, "config1.npz"))
    states = _oracle_trajectory(z)
    print("config1 reset: oracle trajectory done", flush=True)
    w0, b0 = _inputs()
    W = torch.nn.Parameter(w0.to(dev))
    B = torch.nn.Parameter(b0.to(dev))
    opt = Gefen([("weight", W), ("bias", B)], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, factored_v_2d=True)
    worst = []
    for s in range(1, 11):
        prev, ref = states[s - 1], states[s]
        if s > 1:
            sw, sb = opt.state[W], opt.state[B]
            with torch.no_grad():
                W.copy_(torch.from_numpy(prev["W"]).reshape(4096, 4096))
                B.copy_(torch.from_numpy(prev["B"]))
            sw["m_codebook"].copy_(torch.from_numpy(prev["iw"]).reshape(sw["m_codebook"].shape))
            sw["m_magnitude"].copy_(torch.from_numpy(prev["mw"]).reshape(sw["m_magnitude"].shape))
            sw["v_row"].copy_(torch.from_numpy(prev["vr"]))
            sw["v_col"].copy_(torch.from_numpy(prev["vc"]))
            sb["m_codebook"].copy_(torch.from_numpy(prev["ib"]).reshape(sb["m_codebook"].shape))
            sb["m_magnitude"].copy_(torch.from_numpy(prev["mb"]).reshape(sb["m_magnitude"].shape))
            sb["vmean"].copy_(torch.from_numpy(prev["vm"]).reshape(sb["vmean"].shape))
        gw, gb = _inputs(s)
        W.grad, B.grad = gw.to(dev), gb.to(dev)
        opt.step()
        torch.cuda.synchronize()
        sw, sb = opt.state[W], opt.state[B]
        tag = "reset step %d" % s
        if s == 1:
            assert sw["automatic_period"] == int(z["period_weight"])
            np.testing.assert_array_equal(opt._gefen_codebook.cpu().numpy(), z["codebook"])
        np.testing.assert_array_equal(sw["m_codebook"].cpu().numpy().reshape(-1), ref["iw"], err_msg=tag + " W idx")
        np.testing.assert_array_equal(sw["m_magnitude"].cpu().numpy().reshape(-1), ref["mw"], err_msg=tag + " W mag")
        np.testing.assert_allclose(sw["v_row"].cpu().numpy(), ref["vr"], rtol=1e-6, atol=0, err_msg=tag + " v_row")
        np.testing.assert_allclose(sw["v_col"].cpu().numpy(), ref["vc"], rtol=1e-6, atol=0, err_msg=tag + " v_col")
        np.testing.assert_array_equal(sb["m_codebook"].cpu().numpy().reshape(-1), ref["ib"], err_msg=tag + " B idx")
        np.testing.assert_array_equal(sb["m_magnitude"].cpu().numpy().reshape(-1), ref["mb"], err_msg=tag + " B mag")
        np.testing.assert_allclose(sb["vmean"].cpu().numpy().reshape(-1), ref["vm"], rtol=1e-6, atol=0,
                                   err_msg=tag + " vmean")
        for what, got, want in (("W", W.detach().cpu().numpy().reshape(-1), ref["W"].reshape(-1)),
                                ("B", B.detach().cpu().numpy(), ref["B"])):
            err = np.abs(got.astype(np.float64) - want.astype(np.float64))
            lim = 1e-6 * np.abs(want.astype(np.float64))
            bad = err > lim
            rel = err / np.maximum(np.abs(want.astype(np.float64)), 1e-45)
            worst.append((s, what, int(bad.sum()), float(rel.max()), int((err > 0).sum()),
                          float(np.abs(want[np.argmax(rel)]))))
            print("config1 reset step %d %s: %d beyond 1e-6*|p|, worst rel %.3g, %d differ, |p| at worst %.3g"
                  % worst[-1], flush=True)
    failed = [w for w in worst if w[2]]
    assert not failed, "elements beyond 1e-6*|p|: %s" % failed
