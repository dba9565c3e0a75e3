"""Pins of the oracle functions behind the boundary's standalone entry
points: vmean_update, partial_update (the legacy partial update) and
factored_v_ema.

  * Decomposition: the reference's non-fused block step (pinned to its golden
    trajectories, tests/golden/step_block_*.npz) is vmean_update, then the
    host stepsize of gefen.py:3794-3805 (h = sqrt(vmean)/sqrt(bc2) + eps,
    step = (1/h) * (1/bc1)), then partial_update with that stepsize -- so a
    wrong term in either piece breaks bit equality with block_step.
  * factored_v_ema is the correctly rounded fma(1-beta2, RN(sq*RN(1/n)),
    RN(v*beta2)) (checked with exact rational arithmetic), reduces to
    RN(sq*RN(1/n)) at beta2 = 0 and to RN(v*beta2) for zero sums.
"""
import os
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
B1, B2, LR, EPS = 0.9, 0.999, 6e-5, 1e-8
DT = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}


@pytest.mark.parametrize("name", ["block_bf16", "block_f32", "block_f16"])
def test_block_step_is_vmean_then_partial_update(name):
    z = np.load(os.path.join(GOLD, "step_%s.npz" % name))
    dtype = DT[name.split("_")[1]]
    assert float(z["wd"]) >= 0.0
    cb = z["codebook"]
    pnames = sorted({k.split("_", 1)[1] for k in z.files if k.startswith("p0_")})
    for pn in pnames:
        per = int(z["period_" + pn])
        p = z["p0_" + pn]
        nb = p.size // per
        st = {"idx": np.zeros(p.size, np.uint8), "mag": np.zeros(nb, np.float32), "vm": np.zeros(nb, np.float32)}
        for s in range(1, int(z["steps"]) + 1):
            g = z["g%d_%s" % (s, pn)]
            bc1, bc2 = 1 - B1 ** s, 1 - B2 ** s
            p1, i1, m1, v1 = orc.block_step(p, g, st["idx"], st["mag"], st["vm"], per, cb, dtype, beta1=B1, beta2=B2,
                                            lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=0.0)
            vm = orc.vmean_update(st["vm"], g, per, dtype, B2)
            h = (np.sqrt(vm) / np.float32(np.sqrt(bc2)) + np.float32(EPS)).astype(np.float32)
            step = ((np.float32(1.0) / h) * np.float32(1.0 / bc1)).astype(np.float32)
            p2, i2, m2 = orc.partial_update(p, g, st["idx"], st["mag"], step, per, cb, dtype, beta1=B1, lr=LR)
            tag = "%s %s step %d" % (name, pn, s)
            np.testing.assert_array_equal(vm, v1, err_msg=tag)
            np.testing.assert_array_equal(i2, i1, err_msg=tag)
            np.testing.assert_array_equal(m2, m1, err_msg=tag)
            np.testing.assert_array_equal(p2.reshape(-1), p1.reshape(-1), err_msg=tag)
            # and against the reference's own recorded step
            np.testing.assert_array_equal(i2, z["idx%d_%s" % (s, pn)], err_msg=tag)
            p, st = p1, {"idx": i1, "mag": m1, "vm": v1}


def test_partial_update_lr_zero_leaves_p():
    rng = np.random.default_rng(1)
    cb = np.load(os.path.join(GOLD, "learn.npz"))["cb"]
    p = rng.standard_normal(256).astype(np.float32)
    g = (rng.standard_normal(256) * 1e-3).astype(np.float32)
    p1, idx, mag = orc.partial_update(p, g, np.zeros(256, np.uint8), np.zeros(4, np.float32),
                                      np.ones(4, np.float32), 64, cb, orc.F32, beta1=B1, lr=0.0)
    np.testing.assert_array_equal(p1, p)
    assert (mag > 0).all()


def _correctly_rounded_fma(a, b, c):
    """fma(a, b, c) rounded once to fp32, from exact rationals: the fp32 value
    nearest to a*b+c (ties to even)."""
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    guess = np.float32(float(exact))
    cands = [np.nextafter(guess, np.float32(-np.inf)), guess, np.nextafter(guess, np.float32(np.inf))]
    best = min(cands, key=lambda x: (abs(Fraction(float(x)) - exact),
                                     int(np.float32(x).view(np.uint32)) & 1))
    return np.float32(best)


@pytest.mark.parametrize("n", [3, 4096, 14336, 7])
def test_factored_v_ema_is_the_rounded_chain(n):
    rng = np.random.default_rng(n)
    beta2 = 0.999
    v = (np.abs(rng.standard_normal(200)) * np.logspace(-30, 10, 200)).astype(np.float32)
    sq = (rng.standard_normal(200) * np.logspace(-15, 5, 200)).astype(np.float32) ** 2
    got = orc.factored_v_ema(v, sq, n, beta2)
    inv = np.float32(1.0) / np.float32(n)
    a2 = np.float32(1.0 - beta2)
    for i in range(200):
        t = np.float32(sq[i] * inv)
        vb = np.float32(v[i] * np.float32(beta2))
        assert got[i] == _correctly_rounded_fma(a2, t, vb), (i, v[i], sq[i])


def test_factored_v_ema_special_cases():
    rng = np.random.default_rng(2)
    v = np.abs(rng.standard_normal(64)).astype(np.float32)
    sq = np.abs(rng.standard_normal(64)).astype(np.float32)
    inv = np.float32(1.0) / np.float32(96)
    np.testing.assert_array_equal(orc.factored_v_ema(v, sq, 96, 0.0), (sq * inv).astype(np.float32))
    np.testing.assert_array_equal(orc.factored_v_ema(v, np.zeros(64, np.float32), 96, 0.9),
                                  (v * np.float32(0.9)).astype(np.float32))


@pytest.mark.parametrize("bins", [4096, 1024, 256, 2])
def test_histogram_forms_agree_for_power_of_two_bins(bins):
    """The torch path's division by 2/bins and the reference kernel's
    multiply by bins/2 bin every value alike when bins is a power of two (the
    kernel form is thereby pinned wherever the golden codebooks pin the torch
    form)."""
    z = np.load(os.path.join(GOLD, "learn.npz"))
    for key, per in (("g_w", int(z["period_w"])), ("g_b", int(z["period_b"]))):
        a = orc.exact_histogram(z[key], per, bins)
        b = orc.exact_histogram(z[key], per, bins, kernel_scale=True)
        np.testing.assert_array_equal(a, b)
        assert a.sum() == z[key].size


def test_histogram_kernel_form_odd_bins():
    """bins = 37: x = -1 lands in bin 0, x = +1 is clamped into the last
    bin, x = 0 lands in floor(18.5) = 18 (the multiply by bins/2 = 18.5)."""
    g = np.array([-1.0, 1.0, 0.0, 0.5], np.float32)  # one block, absmax 1
    c = orc.exact_histogram(g, 4, 37, kernel_scale=True)
    assert c[0] == 1 and c[36] == 1 and c[18] == 1 and c[int(np.floor(1.5 * 18.5))] == 1


@pytest.mark.parametrize("period", [16, 4096, 1 << 16])
def test_oracle_threads_are_bit_identical(period):
    """The oracle's parallel loops keep each element's operation order:
    factored, block and momentum steps give the same bits on 1 and 4
    threads (many small blocks handed out whole, or few large blocks split)."""
    rng = np.random.default_rng(period)
    cb = np.load(os.path.join(GOLD, "learn.npz"))["cb"]
    rows, cols = 256, 1024
    p = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    g = (rng.standard_normal((rows, cols)) * 1e-3).astype(np.float32)
    idx = rng.integers(0, 256, rows * cols).astype(np.uint8)
    nb = rows * cols // period
    mag = (rng.uniform(0.5, 1.5, nb) * 1e-3).astype(np.float32)
    vr = np.abs(rng.standard_normal(rows) * 1e-6).astype(np.float32)
    vc = np.abs(rng.standard_normal(cols) * 1e-6).astype(np.float32)
    vm = np.abs(rng.standard_normal(nb) * 1e-6).astype(np.float32)
    kw = dict(beta1=B1, beta2=B2, lr=LR, eps=EPS, bc1=0.5, bc2=0.01, wd=0.01)
    outs = []
    for threads in (1, 4):
        orc.set_threads(threads)
        try:
            outs.append((orc.factored_step(p, g, idx, mag, vr, vc, period, cb, orc.BF16, **kw),
                         orc.block_step(p, g, idx, mag, vm, period, cb, orc.F32, **kw),
                         orc.momentum_update(g, idx, mag, period, cb, orc.F16, B1, sr_seed=77)))
        finally:
            orc.set_threads(1)
    for a, b in zip(outs[0], outs[1]):
        for x, y in zip(a, b):
            assert np.asarray(x).tobytes() == np.asarray(y).tobytes()
