"""Pins of oracle.cautious_mask (gefen_muon.py:396-405) by what fixes the
result without restating it: the all-agree and all-disagree cases, an exact
half (scale 2), a scale that rounds (7/3 -> bf16 2.328125), the sign of a
masked zero, and the promotion rule that decides a sign test that underflows
in bf16 but not in fp32."""
import numpy as np

from oracle import oracle as orc


def _bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


def _u(shape, seed=0):
    return orc.bf16(np.random.default_rng(seed).standard_normal(shape).astype(np.float32))


def test_all_agree_is_the_identity():
    u = _u((6, 8))
    out = orc.cautious_mask(u, u * np.float32(3.0), orc.BF16)
    np.testing.assert_array_equal(_bits(out), _bits(u))


def test_nothing_agrees_gives_signed_zeros():
    u = _u((4, 5), 1)
    out = orc.cautious_mask(u, -u, orc.F32)
    assert (out == 0).all()
    np.testing.assert_array_equal(np.signbit(out), np.signbit(u))
    out0 = orc.cautious_mask(u, np.zeros_like(u), orc.BF16)  # a zero gradient agrees with nothing
    assert (out0 == 0).all()


def test_half_agree_doubles_the_rest_exactly():
    u = _u((8, 8), 2)
    g = u.copy()
    g.reshape(-1)[::2] *= -1.0  # every other element disagrees: 32 of 64 agree
    out = orc.cautious_mask(u, g, orc.F32).reshape(-1)
    uf = u.reshape(-1)
    np.testing.assert_array_equal(_bits(out[1::2]), _bits(orc.bf16(uf[1::2] * 2.0)))
    assert (out[::2] == 0).all()


def test_scale_rounds_through_fp32_then_bf16():
    u = orc.bf16(np.array([[1.0, -1.5, 0.75, 2.0, 1.25, -0.5, 3.0]], np.float32))
    # 4 of 7 agree: 7/4 = 1.75 exactly
    g = np.array([[1.0, 1.0, 1.0, -1.0, -1.0, -1.0, 1.0]], np.float32)
    keep = np.array([True, False, True, False, False, True, True])
    out = orc.cautious_mask(u, g, orc.F32)
    np.testing.assert_array_equal(out[0][keep], orc.bf16(u[0][keep] * np.float32(1.75)))
    assert (out[0][~keep] == 0).all()
    # 3 of 7 agree: 7/3 = 2.3333.. is 2.328125 in bf16
    g = np.array([[1.0, 1.0, 1.0, -1.0, 1.0, 1.0, -1.0]], np.float32)
    keep = np.array([True, False, True, False, True, False, False])
    out = orc.cautious_mask(u, g, orc.F32)
    np.testing.assert_array_equal(out[0][keep], orc.bf16(u[0][keep] * np.float32(2.328125)))
    assert (out[0][~keep] == 0).all()


def test_sign_test_takes_the_promoted_dtype():
    tiny = np.float32(2.0 ** -70)  # a product of 2^-140: below bf16's smallest subnormal, an fp32 subnormal
    u = orc.bf16(np.array([[tiny, 1.0]], np.float32))
    g = np.array([[tiny, 1.0]], np.float32)
    out_bf = orc.cautious_mask(u, g, orc.BF16)   # bf16 x bf16 -> bf16: the tiny product is 0, no agreement
    out_f32 = orc.cautious_mask(u, g, orc.F32)   # bf16 x fp32 -> fp32: it agrees
    assert out_bf[0, 0] == 0 and out_bf[0, 1] == np.float32(2.0)
    assert out_f32[0, 0] == tiny and out_f32[0, 1] == np.float32(1.0)
