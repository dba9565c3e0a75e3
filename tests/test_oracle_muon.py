"""The oracle's Muon path against the reference's own CPU step (golden vectors
from tests/golden/make_golden.py): Newton-Schulz, the quantised momentum
recurrence of GefenMuon, NorMuon, the Muon apply and the GefenMuonHybrid
routing.  CPU only."""
import os

import numpy as np
import pytest

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = {"bf16": orc.BF16, "f32": orc.F32}


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


def ulp(x, dtype):
    """Spacing of the dtype's values at |x| (bf16: 8-bit significand)."""
    bits = 7 if dtype == orc.BF16 else (10 if dtype == orc.F16 else 23)
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - bits)


def assert_within_ulp(got, ref, dtype, n=1, msg="", atol=0.0):
    """|got - ref| <= n ulps of the dtype at max(|got|, |ref|) + atol."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    lim = n * ulp(np.maximum(np.abs(got), np.abs(ref)), dtype) + atol
    bad = np.abs(got - ref) > lim
    assert not bad.any(), "%s: %d of %d elements beyond %d ulp (max |d| %.3e)" % (
        msg, int(bad.sum()), bad.size, n, float(np.abs(got - ref).max()))


@pytest.mark.parametrize("name", ["wide", "tall", "square", "zero"])
def test_newton_schulz_matches_reference(name):
    z = _load("muon_ns.npz")
    sched = z["abc_" + name] if "abc_" + name in z else None
    got = orc.newton_schulz(z["in_" + name], sched)
    ref = z["out_" + name]
    assert got.shape == ref.shape
    # same op order and roundings; the GEMMs sum in a different order, so a
    # rare element may land one bf16 ulp away
    assert np.mean(got == ref) >= 0.999
    np.testing.assert_allclose(got, ref, rtol=2.0 ** -7, atol=2.0 ** -12)


def test_newton_schulz_tuned_schedule_close():
    z = _load("muon_ns.npz")
    got = orc.newton_schulz(z["in_wide4"], z["abc_wide4"])
    ref = z["out_wide4"]
    assert np.linalg.norm(got - ref) <= 1e-2 * np.linalg.norm(ref)


def test_newton_schulz_orthogonalises():
    """Closed-form check independent of the reference: after 10 standard
    iterations the singular values sit in the quintic's band (0.5, 1.3)
    (the reference's own band, tests/test_validation_cpu.py:262-276)."""
    rng = np.random.default_rng(0)
    m = rng.standard_normal((32, 48)).astype(np.float32)
    o = orc.newton_schulz(m, orc.NS_STANDARD * 2)
    s = np.linalg.svd(o.astype(np.float64), compute_uv=False)
    assert s.min() > 0.5 and s.max() < 1.3


def _muon_trajectory(z, names, dtype, beta, nesterov, lr, wd, fn, use_normuon, steps, schedule=None):
    cb = z["codebook"]
    state = {}
    for n in names:
        p0 = z["p0_" + n]
        per = int(z["period_" + n])
        state[n] = dict(p=p0.copy(), idx=np.zeros(p0.size, np.uint8), mag=np.zeros(p0.size // per, np.float32),
                        per=per, v=np.zeros(p0.shape[0], np.float32), nstep=0)
    for s in range(1, steps + 1):
        for n in names:
            st = state[n]
            g = z["g%d_%s" % (s, n)]
            st["idx"], st["mag"], mom = orc.muon_momentum(g, st["idx"], st["mag"], st["per"], cb, dtype, beta,
                                                         nesterov)
            ortho = orc.newton_schulz(mom.reshape(g.shape), schedule)
            if use_normuon:
                st["nstep"] += 1
                ortho, st["v"] = orc.normuon(ortho, st["v"], st["nstep"])
            adj = lr * orc.adjust_lr_ratio(fn, g.shape)
            st["p_prev"] = st["p"]
            st["p"] = orc.muon_apply(st["p"], ortho, dtype, lr, wd, adj)
            yield s, n, st


# Newton-Schulz amplifies rounding differences in the small singular
# directions (the quintic's slope at 0 is a = 3.4445, so 5 iterations scale
# them by ~480): two correct implementations whose GEMMs sum in different
# orders agree only to the reference's own bound between its batched and
# serial paths, rel-L2 <= 2e-2 (tests/test_batched_ns.py:56-71).
NS_REL = 2e-2


def assert_update_close(got, ref, adj, dtype, msg):
    """New parameters (same starting p) differ by at most adj * (NS
    difference) plus p's own rounding: ||got - ref|| <= adj * NS_REL * ||ortho||
    + ||ulp(p)||, with ||ortho||_F <= 1.3 * sqrt(min(R, C)) (singular values of
    the NS output lie below 1.3)."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    ortho_norm = 1.3 * np.sqrt(min(got.shape))
    lim = adj * NS_REL * ortho_norm + np.linalg.norm(ulp(np.maximum(np.abs(got), np.abs(ref)), dtype))
    d = np.linalg.norm(got - ref)
    assert d <= lim, "%s: ||dp|| %.3e > %.3e" % (msg, d, lim)


@pytest.mark.parametrize("case", ["muon_bf16", "muon_f32"])
def test_muon_trajectory_matches_reference(case):
    z = _load(case + ".npz")
    if case == "muon_bf16":
        kw = dict(dtype=orc.BF16, beta=0.95, nesterov=True, lr=0.02, wd=0.1, fn=None, use_normuon=False, steps=4)
    else:
        kw = dict(dtype=orc.F32, beta=0.9, nesterov=False, lr=0.02, wd=0.1, fn="match_rms_adamw",
                  use_normuon=True, steps=3)
    prev = {n: z["p0_" + n] for n in ("a", "b")}
    for s, n, st in _muon_trajectory(z, ["a", "b"], **kw):
        tag = "%s step %d %s" % (case, s, n)
        # the quantised momentum never sees Newton-Schulz: bit-exact
        np.testing.assert_array_equal(st["idx"], z["idx%d_%s" % (s, n)], err_msg=tag + " indices")
        np.testing.assert_array_equal(st["mag"], z["mag%d_%s" % (s, n)], err_msg=tag + " magnitudes")
        adj = kw["lr"] * orc.adjust_lr_ratio(kw["fn"], z["p0_" + n].shape)
        ref_p = z["p%d_%s" % (s, n)]
        # both steps start from the reference's previous parameters
        assert_update_close(st["p"], ref_p, adj, kw["dtype"], tag + " params")
        prev[n] = ref_p
        st["p"] = ref_p.copy()  # continue from the reference's parameters
        if "nv%d_%s" % (s, n) in z:
            nv_ref = z["nv%d_%s" % (s, n)]
            assert np.linalg.norm(st["v"] - nv_ref) <= 2 * NS_REL * np.linalg.norm(nv_ref), tag + " normuon_v"
            st["v"] = nv_ref.copy()


TUNED3 = [(5.0067, -14.4125, 10.6001), (3.7534, -6.8083, 3.3840), (3.2080, -4.3501, 2.0330)]


def test_hybrid_trajectory_matches_reference():
    """GefenMuonHybrid defaults (hybrid.py:228-265): Muon with the tuned
    3-step schedule, match_rms_adamw and NorMuon; the embedding and the norm
    vector take the block-vmean Gefen backup."""
    z = _load("hybrid_bf16.npz")
    cb = z["codebook"]
    lr, wd = 1e-3, 0.01
    muon = ["layers.0.mlp.w", "layers.0.attn.o"]
    backup = ["embed_tokens.weight", "layers.0.norm.weight"]
    st = {}
    for n in muon + backup:
        p0 = z["p0_" + n]
        per = int(z["period_" + n])
        st[n] = dict(p=p0.copy(), idx=np.zeros(p0.size, np.uint8), mag=np.zeros(p0.size // per, np.float32),
                     per=per, v=np.zeros(p0.shape[0], np.float32), vmean=np.zeros(p0.size // per, np.float32))
    for s in range(1, 4):
        for n in backup:  # the backup steps first (hybrid.py:760-763)
            t = st[n]
            g = z["g%d_%s" % (s, n)].reshape(-1)
            p, idx, mag, vm = orc.block_step(t["p"].reshape(-1), g, t["idx"], t["mag"], t["vmean"], t["per"], cb,
                                             orc.BF16, beta1=0.9, beta2=0.999, lr=lr, eps=1e-8,
                                             bc1=1 - 0.9 ** s, bc2=1 - 0.999 ** s, wd=wd)
            tag = "hybrid step %d %s" % (s, n)
            np.testing.assert_array_equal(idx, z["idx%d_%s" % (s, n)], err_msg=tag)
            np.testing.assert_array_equal(mag, z["mag%d_%s" % (s, n)], err_msg=tag)
            np.testing.assert_allclose(vm, z["vmean%d_%s" % (s, n)], rtol=1e-6, err_msg=tag)
            assert_within_ulp(p, z["p%d_%s" % (s, n)].reshape(-1), orc.BF16, 1, tag)
            t.update(p=p.reshape(t["p"].shape), idx=idx, mag=mag, vmean=vm)
        for n in muon:
            t = st[n]
            g = z["g%d_%s" % (s, n)]
            tag = "hybrid step %d %s" % (s, n)
            t["idx"], t["mag"], mom = orc.muon_momentum(g, t["idx"], t["mag"], t["per"], cb, orc.BF16, 0.95, True)
            np.testing.assert_array_equal(t["idx"], z["idx%d_%s" % (s, n)], err_msg=tag)
            np.testing.assert_array_equal(t["mag"], z["mag%d_%s" % (s, n)], err_msg=tag)
            ortho = orc.newton_schulz(mom.reshape(g.shape), TUNED3)
            ortho, v = orc.normuon(ortho, t["v"], s)
            nv_ref = z["normuon_v%d_%s" % (s, n)]
            assert np.linalg.norm(v - nv_ref) <= 2 * NS_REL * np.linalg.norm(nv_ref), tag + " normuon_v"
            adj = lr * orc.adjust_lr_ratio("match_rms_adamw", g.shape)
            p = orc.muon_apply(t["p"], ortho, orc.BF16, lr, wd, adj)
            ref_p = z["p%d_%s" % (s, n)]
            assert_update_close(p, ref_p, adj, orc.BF16, tag + " params")
            t.update(p=ref_p.copy(), v=nv_ref.copy())
