"""Pins of the oracle's stochastic rounding (oracle.sr_uniform / sr_quantize
and the sr_seed form of the step functions), restating
kernels/automatic_gefen_fused_kernel.cu:141-151 (the SplitMix64 finalizer
over seed + gamma * (element + 1), top 24 bits) and :160-211 / :273-328 (round
to one of the two bracketing codewords, up with probability
(x - lo) / (hi - lo)).  The reference's CPU step has no stochastic rounding,
so no golden trajectory exists; these checks fix it instead:
  - published SplitMix64 outputs: the uniform for (seed, element i) is the
    top 24 bits of output i of the SplitMix64 stream seeded with `seed`;
  - exact codewords, the codebook ends, out-of-range and NaN inputs;
  - only the two bracketing codewords are ever chosen;
  - unbiasedness: the mean of c[idx] over many draws equals x.
"""
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# Published SplitMix64 outputs (the generator's reference sequence):
#   seed 0:       the first three outputs of the stream;
#   seed 1234567: the first five (Rosetta Code, "Pseudo-random numbers/Splitmix64").
SPLITMIX64_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
SPLITMIX64_SEED1234567 = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                          4593380528125082431, 16408922859458223821]


def _cb():
    return np.load(os.path.join(GOLD, "learn.npz"))["cb"].astype(np.float32)


@pytest.mark.parametrize("seed,outputs", [(0, SPLITMIX64_SEED0), (1234567, SPLITMIX64_SEED1234567)])
def test_sr_uniform_is_splitmix64_stream(seed, outputs):
    for i, z in enumerate(outputs):
        assert orc.sr_uniform(seed, i) == (z >> 40) / float(1 << 24), (seed, i)


def test_sr_uniform_range_and_resolution():
    us = np.array([orc.sr_uniform(7, i) for i in range(4096)])
    assert us.min() >= 0.0 and us.max() < 1.0
    assert np.all(us * (1 << 24) == np.floor(us * (1 << 24)))  # multiples of 2^-24


def test_sr_exact_codewords_and_ends():
    cb = _cb()
    k = cb.size
    for seed in (0, 1, 99, 2 ** 63 + 5):
        for j in range(k):
            assert orc.sr_quantize(cb, float(cb[j]), seed, j) == j
        assert orc.sr_quantize(cb, -1.0, seed, 3) == 0
        assert orc.sr_quantize(cb, 1.0, seed, 3) == k - 1
        assert orc.sr_quantize(cb, 1.5, seed, 3) == k - 1      # beyond the top end: clamped up
        assert orc.sr_quantize(cb, -1.5, seed, 3) == 0         # below the bottom end
        assert orc.sr_quantize(cb, float("nan"), seed, 3) == 0
    one = np.array([0.25], np.float32)
    assert orc.sr_quantize(one, 0.7, 3, 0) == 0


def test_sr_picks_a_bracketing_codeword():
    cb = _cb()
    rng = np.random.default_rng(0)
    xs = rng.uniform(-1, 1, 400).astype(np.float32)
    for e, x in enumerate(xs):
        r = int(np.searchsorted(cb, x, side="left"))
        got = orc.sr_quantize(cb, float(x), 11, e)
        assert got in (r - 1, r), (x, got, r)


def test_sr_is_unbiased():
    """E[c[idx]] = x: over N draws the mean of c[idx] is within 6 sigma of x,
    sigma <= (hi - lo) / (2 sqrt(N)).  A flipped comparison (rounding up
    with probability 1 - p_up) or a swapped bracket fails this."""
    cb = _cb()
    n = 20000
    for x, seed in ((0.0123, 5), (-0.3337, 6), (0.91, 7), (-0.999, 8)):
        r = int(np.searchsorted(cb, np.float32(x), side="left"))
        lo, hi = float(cb[r - 1]), float(cb[r])
        vals = np.array([cb[orc.sr_quantize(cb, x, seed, e)] for e in range(n)], np.float64)
        sigma = (hi - lo) / (2.0 * np.sqrt(n))
        assert abs(vals.mean() - x) < 6 * sigma, (x, vals.mean(), sigma)
        p_up = (np.float32(x) - np.float32(lo)) / (np.float32(hi) - np.float32(lo))
        frac_up = np.mean(vals == hi)
        assert abs(frac_up - p_up) < 6 * np.sqrt(p_up * (1 - p_up) / n) + 1e-12


def test_sr_step_uses_flat_element_index():
    """The sr_seed form of the momentum update requantises element e of the
    tensor with sr_quantize(x_e, seed, e), where x_e is the nearest path's
    normalised value u_e / mag'_b (the magnitudes do not depend on the
    rounding)."""
    cb = _cb()
    rng = np.random.default_rng(3)
    period, nb = 96, 5
    g = (rng.standard_normal(period * nb) * 1e-3).astype(np.float32)
    idx0 = rng.integers(0, 256, period * nb).astype(np.uint8)
    mag0 = (rng.uniform(0.5, 1.5, nb) * 1e-3).astype(np.float32)
    i_n, m_n, _, u = orc.momentum_update(g, idx0, mag0, period, cb, orc.F32, 0.9)
    i_s, m_s, q_s, _ = orc.momentum_update(g, idx0, mag0, period, cb, orc.F32, 0.9, sr_seed=1234)
    np.testing.assert_array_equal(m_s, m_n)
    x = (u.reshape(nb, period) / m_n[:, None]).astype(np.float32).reshape(-1)
    want = np.array([orc.sr_quantize(cb, float(x[e]), 1234, e) for e in range(x.size)], np.uint8)
    np.testing.assert_array_equal(i_s, want)
    assert (i_s != i_n).any()
    np.testing.assert_array_equal(q_s, (cb[i_s] * np.repeat(m_s, period)).astype(np.float32))
    # the nearest mode is restored after an sr_seed call
    i_n2, _, _, _ = orc.momentum_update(g, idx0, mag0, period, cb, orc.F32, 0.9)
    np.testing.assert_array_equal(i_n2, i_n)
