"""Pin the C oracle against the reference's own outputs (tests/golden/*.npz).

The fixtures were written by tests/golden/make_golden.py, which ran the
reference's CPU path read-only in the build container.  These tests need no
GPU and never touch the reference.
"""
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    path = os.path.join(GOLD, name)
    if not os.path.exists(path):
        pytest.skip("golden fixture %s not generated" % name)
    return np.load(path)


@pytest.mark.parametrize("tag", ["k256", "k1", "k2", "k3"])
def test_nearest_matches_reference(tag):
    z = _load("nearest.npz")
    got = orc.nearest_indices(z["cb_" + tag], z["x_" + tag])
    np.testing.assert_array_equal(got, z["idx_" + tag])


@pytest.mark.parametrize("tag", ["rand", "dense", "k3"])
def test_search_lut_matches_reference(tag):
    z = _load("lut.npz")
    np.testing.assert_array_equal(orc.search_lut(z["cb_" + tag]), z["lut_" + tag])


@pytest.mark.parametrize("tag", ["pad40", "a300", "a520"])
def test_exact_dp_matches_reference(tag):
    z = _load("dp.npz")
    centers, counts = orc.histogram_stats(z["counts_" + tag])
    cb = orc.exact_dp(centers, counts)
    np.testing.assert_array_equal(cb, z["cb_" + tag])


def test_learned_codebook_matches_reference():
    z = _load("learn.npz")
    cb = orc.learn_codebook([(z["g_w"], int(z["period_w"])), (z["g_b"], int(z["period_b"]))])
    np.testing.assert_array_equal(cb, z["cb"])


def test_period_search_matches_reference():
    z = _load("period.npz")
    tags = sorted(k[2:] for k in z.files if k.startswith("g_"))
    assert tags
    for tag in tags:
        g = z["g_" + tag]
        period, results = orc.find_period(g, g.shape, return_errors=True)
        np.testing.assert_allclose([e for _, e in results], z["errs_" + tag], rtol=1e-12)
        assert period == int(z["period_" + tag]), tag


STEP_CASES = ["fact_f32", "fact_bf16", "fact_f16", "block_bf16", "block_f32",
              "block_f16", "zeros_f32"]
DTYPE_OF = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}
BETA1, BETA2, LR, EPS = 0.9, 0.999, 6e-5, 1e-8


def _p_tol(dtype):
    # fp32: <= 1e-6 relative; half types: <= 1 ulp of the stored value
    return {orc.F32: 1e-6, orc.BF16: 2.0 ** -7, orc.F16: 2.0 ** -10}[dtype]


def _oracle_step(z, name, pn, s, prev, dtype):
    per = int(z["period_" + pn])
    g = z["g%d_%s" % (s, pn)]
    bc1 = 1 - BETA1 ** s
    bc2 = 1 - BETA2 ** s
    wd = float(z["wd"])
    cb = z["codebook"]
    if int(z["factored"]) and g.ndim == 2:
        p, idx, mag, vr, vc = orc.factored_step(
            prev["p"], g, prev["idx"], prev["mag"], prev["v_row"], prev["v_col"], per,
            cb, dtype, beta1=BETA1, beta2=BETA2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=wd)
        return {"p": p, "idx": idx, "mag": mag, "v_row": vr, "v_col": vc}
    p, idx, mag, vm = orc.block_step(
        prev["p"], g, prev["idx"], prev["mag"], prev["vmean"], per, cb, dtype,
        beta1=BETA1, beta2=BETA2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=wd)
    return {"p": p, "idx": idx, "mag": mag, "vmean": vm}


def _initial_state(z, pn):
    p0 = z["p0_" + pn]
    per = int(z["period_" + pn])
    nb = p0.size // per
    st = {"p": p0, "idx": np.zeros(p0.size, np.uint8), "mag": np.zeros(nb, np.float32)}
    if int(z["factored"]) and p0.ndim == 2:
        st["v_row"] = np.zeros(p0.shape[0], np.float32)
        st["v_col"] = np.zeros(p0.shape[1], np.float32)
    else:
        st["vmean"] = np.zeros(nb, np.float32)
    return st


def _reference_state(z, pn, s):
    st = {"p": z["p%d_%s" % (s, pn)], "idx": z["idx%d_%s" % (s, pn)],
          "mag": z["mag%d_%s" % (s, pn)]}
    for key in ("v_row", "v_col", "vmean"):
        k = "%s%d_%s" % (key, s, pn)
        if k in z.files:
            st[key] = z[k]
    return st


@pytest.mark.parametrize("name", STEP_CASES)
def test_step_trajectory_matches_reference(name):
    """Each step restarts from the reference's previous state, so every
    comparison is a one-step check; indices and magnitudes must be exact."""
    z = _load("step_%s.npz" % name)
    dtype = DTYPE_OF[name.split("_")[1]]
    pnames = sorted({k.split("_", 1)[1] for k in z.files if k.startswith("p0_")})
    steps = int(z["steps"])
    for pn in pnames:
        prev = _initial_state(z, pn)
        for s in range(1, steps + 1):
            got = _oracle_step(z, name, pn, s, prev, dtype)
            ref = _reference_state(z, pn, s)
            np.testing.assert_array_equal(got["idx"], ref["idx"], err_msg="%s idx step %d" % (pn, s))
            np.testing.assert_array_equal(got["mag"], ref["mag"], err_msg="%s mag step %d" % (pn, s))
            for key in ("v_row", "v_col", "vmean"):
                if key in ref:
                    np.testing.assert_allclose(got[key], ref[key], rtol=1e-6, atol=0,
                                               err_msg="%s %s step %d" % (pn, key, s))
            np.testing.assert_allclose(got["p"], ref["p"].reshape(got["p"].shape),
                                       rtol=_p_tol(dtype), atol=1e-30,
                                       err_msg="%s p step %d" % (pn, s))
            prev = {k: np.asarray(v).copy() for k, v in ref.items()}
            prev["p"] = prev["p"].reshape(z["p0_" + pn].shape)


@pytest.mark.parametrize("name", STEP_CASES)
def test_free_running_indices_match_reference(name):
    """Free-running oracle trajectory: indices stay bit-exact for every step."""
    z = _load("step_%s.npz" % name)
    dtype = DTYPE_OF[name.split("_")[1]]
    pnames = sorted({k.split("_", 1)[1] for k in z.files if k.startswith("p0_")})
    for pn in pnames:
        st = _initial_state(z, pn)
        for s in range(1, int(z["steps"]) + 1):
            st = _oracle_step(z, name, pn, s, st, dtype)
            np.testing.assert_array_equal(st["idx"], z["idx%d_%s" % (s, pn)])


# ------------------------------------------------------------------ config 1

def config1_inputs(step=None):
    """BASELINE config 1 inputs, the seed protocol tests/golden/make_golden.py
    used: W 4096x4096 and b 4096 fp32 ~ N(0, 0.02) from seed 0; the step-t
    grads ~ N(0, 1e-3) from seed 1000 + t (W's first, then b's)."""
    import torch
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(4096, 4096, generator=gen) * 0.02
    b = torch.randn(4096, generator=gen) * 0.02
    if step is None:
        return w.numpy(), b.numpy()
    gt = torch.Generator().manual_seed(1000 + step)
    return ((torch.randn(4096, 4096, generator=gt) * 1e-3).numpy(),
            (torch.randn(4096, generator=gt) * 1e-3).numpy())


C1_SUB = 4099  # subsample stride of the golden weight snapshots
C1_WD = 0.01


def _sha(a):
    import hashlib
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _assert_p_close(got, ref, p0, what):
    scale = np.maximum(np.abs(p0), np.abs(ref)).astype(np.float64)
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    bad = err > 1e-6 * scale
    assert not bad.any(), "%s: %d elements beyond 1e-6 of max(|p0|,|p|), worst %.3g" % (
        what, int(bad.sum()), float((err / np.maximum(scale, 1e-38)).max()))


def test_config1_trajectory_matches_reference():
    """the reference's CPU step (fused=False, factored)
    on a 4096x4096 fp32 weight plus a 4096 bias for 10 steps.  Step 1 learns
    the period of each tensor and the codebook from the step-1 grads; the
    oracle free-runs the whole trajectory.  Per step: the sha256 of the full
    4096x4096 index array and the magnitudes bit-exact, v_row / v_col / vmean
    within 1e-6 relative (torch's CPU reductions sum in another order), the
    weight subsample and the bias within 1e-6 of max(|p0|, |p|) per element:
    a last-bit difference in a stepsize flips one rounding of p, and that
    ulp (taken while |p| was near |p0|) is carried along even where p later
    shrinks.  Measured: at most 2 ulps of that scale after 10 steps."""
    z = _load("config1.npz")
    w, b = config1_inputs()
    w0_sub, b0 = w.reshape(-1)[::C1_SUB].copy(), b.copy()
    gw, gb = config1_inputs(1)
    pw = orc.resolve_period(gw, gw.shape)
    pb = orc.resolve_period(gb, gb.shape)
    assert (pw, pb) == (int(z["period_weight"]), int(z["period_bias"]))
    cb = orc.learn_codebook([(gw, pw), (gb, pb)])
    np.testing.assert_array_equal(cb, z["codebook"])
    sw = {"idx": np.zeros(w.size, np.uint8), "mag": np.zeros(w.size // pw, np.float32),
          "v_row": np.zeros(4096, np.float32), "v_col": np.zeros(4096, np.float32)}
    sb = {"idx": np.zeros(b.size, np.uint8), "mag": np.zeros(b.size // pb, np.float32),
          "vmean": np.zeros(b.size // pb, np.float32)}
    for s in range(1, 11):
        if s > 1:
            gw, gb = config1_inputs(s)
        bc1, bc2 = 1 - BETA1 ** s, 1 - BETA2 ** s
        w, sw["idx"], sw["mag"], sw["v_row"], sw["v_col"] = orc.factored_step(
            w, gw, sw["idx"], sw["mag"], sw["v_row"], sw["v_col"], pw, cb, orc.F32,
            beta1=BETA1, beta2=BETA2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=C1_WD)
        b, sb["idx"], sb["mag"], sb["vmean"] = orc.block_step(
            b, gb, sb["idx"], sb["mag"], sb["vmean"], pb, cb, orc.F32,
            beta1=BETA1, beta2=BETA2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=C1_WD)
        assert _sha(sw["idx"]) == str(z["sha_idx%d_weight" % s]), "weight indices, step %d" % s
        np.testing.assert_array_equal(sw["idx"][::C1_SUB], z["idx_sub%d_weight" % s])
        np.testing.assert_array_equal(sw["mag"], z["mag%d_weight" % s])
        np.testing.assert_allclose(sw["v_row"], z["v_row%d_weight" % s], rtol=1e-6, atol=0)
        np.testing.assert_allclose(sw["v_col"], z["v_col%d_weight" % s], rtol=1e-6, atol=0)
        _assert_p_close(w.reshape(-1)[::C1_SUB], z["p_sub%d_weight" % s], w0_sub, "weight step %d" % s)
        np.testing.assert_array_equal(sb["idx"], z["idx%d_bias" % s])
        np.testing.assert_array_equal(sb["mag"], z["mag%d_bias" % s])
        np.testing.assert_allclose(sb["vmean"], z["vmean%d_bias" % s], rtol=1e-6, atol=0)
        _assert_p_close(b, z["p%d_bias" % s], b0, "bias step %d" % s)
