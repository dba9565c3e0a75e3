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
