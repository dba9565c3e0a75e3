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
