"""Local oracle checks of one optimizer step on tensors too large for the
oracle to step whole (test helper, imported by the full-size GPU tests).

What is local in the step (gefen.py:2959-3018, 3329-3486, 3776-3818):
  - a block's new indices and magnitude depend only on that block's grads,
    stored indices and old magnitude (oracle.momentum_update, bit-exact);
  - a row's v_row only on that row's grads and old v_row, a column's v_col
    only on that column (the EMA v <- fma(mean(g^2), 1-beta2, v*beta2));
  - an element's new value only on its own p, its block's new index and
    magnitude, v_row of its row, v_col of its column and mean(v_row).
`FactoredProbe.capture` copies those inputs before the step and
`FactoredProbe.verify` checks the GPU's results after it.
"""
from __future__ import annotations

import numpy as np
import torch

from oracle import oracle as orc

TDT_CODE = {torch.float32: orc.F32, torch.float16: orc.F16, torch.bfloat16: orc.BF16}
ULP_RTOL = {orc.F32: 1e-6, orc.F16: 2.0 ** -10, orc.BF16: 2.0 ** -8}


def _f(t):
    return t.detach().float().cpu().numpy()


def assert_within_ulp(got, ref, dtype, msg, atol=0.0):
    """Half types: |got - ref| <= 1 ulp of ref in that dtype (exact spacing
    of the stored value's binade, so 1 ulp means 1 ulp, also at the top of a
    binade), plus `atol`; fp32: 1e-6 relative per element with no absolute
    allowance (`atol` ignored: the fp32 step rounds in the reference's op
    order, so even elements that cancel towards zero agree)."""
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    err = np.abs(got - ref)
    if dtype == orc.F32:
        atol = 0.0
        lim = 1e-6 * np.abs(ref)
    else:
        mant = 7 if dtype == orc.BF16 else 10
        mag = np.abs(ref)
        # spacing of the dtype at |ref| (normal numbers; subnormals use the
        # smallest normal's spacing)
        emin = -126 if dtype == orc.BF16 else -14
        e = np.floor(np.log2(np.where(mag > 0, mag, 1.0)))
        e = np.maximum(e, emin)
        lim = np.where(mag > 0, 2.0 ** (e - mant), 2.0 ** (emin - mant))
    bad = err > lim + atol
    assert not bad.any(), "%s: %d of %d elements beyond 1 ulp (worst err %.3g at ref %.6g)" % (
        msg, int(bad.sum()), err.size, float(err[bad].max()), float(ref[bad][np.argmax(err[bad])]))


class FactoredProbe:
    """Sampled blocks, rows and columns of one 2D factored parameter."""

    def __init__(self, name, p, period, rows, cols, blocks):
        self.name, self.p, self.P = name, p, int(period)
        R, C = p.shape
        self.R, self.C = R, C
        self.rows = sorted({int(r) % R for r in rows})
        self.cols = sorted({int(c) % C for c in cols})
        nb = p.numel() // self.P
        self.blocks = sorted({int(b) % nb for b in blocks})
        self.dtype = TDT_CODE[p.dtype]

    def capture(self, state):
        p, g, P = self.p, self.p.grad, self.P
        fresh = state is None or "step" not in state
        self.p_rows = _f(p[self.rows])
        self.g_cols = _f(g[:, self.cols]).T.copy()
        self.g_rows = _f(g[self.rows])
        self.vr_old = (np.zeros(len(self.rows), np.float32) if fresh
                       else state["v_row"][self.rows].cpu().numpy())
        self.vc_old = (np.zeros(len(self.cols), np.float32) if fresh
                       else state["v_col"][self.cols].cpu().numpy())
        gf = g.reshape(-1)
        self.blk_in = []
        for b in self.blocks:
            gb = _f(gf[b * P:(b + 1) * P])
            ib = np.zeros(P, np.uint8) if fresh else state["m_codebook"].reshape(-1)[b * P:(b + 1) * P].cpu().numpy()
            mb = np.zeros(1, np.float32) if fresh else state["m_magnitude"].reshape(-1)[b:b + 1].cpu().numpy()
            self.blk_in.append((gb, ib, mb))

    @staticmethod
    def _ema(sum_sq64, n, v_old, beta2):
        ms = np.float32(np.float32(sum_sq64) / np.float32(n))
        return np.float32(np.float64(ms) * np.float64(np.float32(1 - beta2)) +
                          np.float64(np.float32(np.float32(v_old) * np.float32(beta2))))

    def verify(self, state, codebook, *, step, beta1, beta2, lr, eps, wd, bc2_step=None):
        P, dt, tag = self.P, self.dtype, "%s step %d" % (self.name, step)
        idx_all = state["m_codebook"].reshape(-1)
        mag_all = state["m_magnitude"].reshape(-1)
        for b, (gb, ib, mb) in zip(self.blocks, self.blk_in):
            i1, m1, _, _ = orc.momentum_update(gb, ib, mb, P, codebook, dt, beta1)
            np.testing.assert_array_equal(idx_all[b * P:(b + 1) * P].cpu().numpy(), i1,
                                          err_msg="%s block %d indices" % (tag, b))
            np.testing.assert_array_equal(mag_all[b:b + 1].cpu().numpy(), m1,
                                          err_msg="%s block %d magnitude" % (tag, b))
        v_row = state["v_row"].cpu().numpy()
        v_col = state["v_col"].cpu().numpy()
        for j, r in enumerate(self.rows):
            ref = self._ema(np.sum(self.g_rows[j].astype(np.float64) ** 2), self.C, self.vr_old[j], beta2)
            np.testing.assert_allclose(v_row[r], ref, rtol=1e-6, err_msg="%s v_row[%d]" % (tag, r))
        for j, c in enumerate(self.cols):
            ref = self._ema(np.sum(self.g_cols[j].astype(np.float64) ** 2), self.R, self.vc_old[j], beta2)
            np.testing.assert_allclose(v_col[c], ref, rtol=1e-6, err_msg="%s v_col[%d]" % (tag, c))
        # elements of the sampled rows from the GPU's own v and new state
        bc1 = 1 - beta1 ** step
        bc2 = 1 - beta2 ** (step if bc2_step is None else bc2_step)
        mean = np.float32(np.sum(v_row.astype(np.float64)) / self.R)
        cbd = orc.round_dtype(np.asarray(codebook, np.float32), dt)
        for j, r in enumerate(self.rows):
            flat = np.arange(r * self.C, (r + 1) * self.C)
            idx_r = idx_all[r * self.C:(r + 1) * self.C].cpu().numpy()
            ub, inv = np.unique(flat // P, return_inverse=True)
            mags = mag_all[torch.from_numpy(ub).to(mag_all.device)].cpu().numpy()[inv]
            q = (cbd[idx_r] * mags.astype(np.float32)).astype(np.float32)
            vh = (np.float32(v_row[r]) * v_col) / mean
            h = np.sqrt(vh / np.float32(bc2)) + np.float32(eps)
            stp = (np.float32(1.0) / h) * np.float32(1.0 / bc1)
            pw = self.p_rows[j]
            if wd > 0:
                pw = orc.round_dtype((pw * np.float32(1 - lr * wd)).astype(np.float32), dt)
            p_ref = orc.round_dtype((pw - (q * stp) * np.float32(lr)).astype(np.float32), dt)
            # 1 ulp plus 1e-6 * lr: the stepsize carries the summation-order
            # skew of v (1e-6 relative), visible where p cancels towards zero
            assert_within_ulp(_f(self.p[r]), p_ref, dt, "%s row %d p" % (tag, r), atol=1e-6 * lr)


class BlockProbe:
    """Sampled momentum blocks of one block-vmean (factored_v_2d off or 1D)
    parameter.  Blocks are independent on this path (gefen.py:3776-3818): a
    block's new indices, magnitude, vmean and parameters depend only on its
    own p, grad, indices, magnitude and vmean, so oracle.block_step over the
    block alone gives its exact step."""

    def __init__(self, name, p, period, blocks):
        self.name, self.p, self.P = name, p, int(period)
        nb = p.numel() // self.P
        self.blocks = sorted({int(b) % nb for b in blocks})
        self.dtype = TDT_CODE[p.dtype]

    def capture(self, state):
        P = self.P
        pf = self.p.detach().reshape(-1)
        gf = self.p.grad.reshape(-1)
        idx = state["m_codebook"].reshape(-1)
        mag = state["m_magnitude"].reshape(-1)
        vm = state["vmean"].reshape(-1)
        self.blk_in = [(_f(pf[b * P:(b + 1) * P]), _f(gf[b * P:(b + 1) * P]),
                        idx[b * P:(b + 1) * P].cpu().numpy(), mag[b:b + 1].cpu().numpy(),
                        vm[b:b + 1].cpu().numpy()) for b in self.blocks]

    def verify(self, state, codebook, *, step, beta1, beta2, lr, eps, wd, bc2_step=None):
        P, tag = self.P, "%s step %d" % (self.name, step)
        bc1 = 1 - beta1 ** step
        bc2 = 1 - beta2 ** (step if bc2_step is None else bc2_step)
        pf = self.p.detach().reshape(-1)
        idx = state["m_codebook"].reshape(-1)
        mag = state["m_magnitude"].reshape(-1)
        vm = state["vmean"].reshape(-1)
        for b, (p0, g0, i0, m0, v0) in zip(self.blocks, self.blk_in):
            p1, i1, m1, v1 = orc.block_step(p0, g0, i0, m0, v0, P, codebook, self.dtype, beta1=beta1, beta2=beta2,
                                            lr=lr, eps=eps, bc1=bc1, bc2=bc2, wd=wd)
            btag = "%s block %d" % (tag, b)
            np.testing.assert_array_equal(idx[b * P:(b + 1) * P].cpu().numpy(), i1, err_msg=btag + " indices")
            np.testing.assert_array_equal(mag[b:b + 1].cpu().numpy(), m1, err_msg=btag + " magnitude")
            np.testing.assert_allclose(vm[b:b + 1].cpu().numpy(), v1, rtol=1e-6, err_msg=btag + " vmean")
            assert_within_ulp(_f(pf[b * P:(b + 1) * P]), p1, self.dtype, btag + " p", atol=1e-6 * lr)


def ns_torch_fp32(m, sched, eps=1e-7):
    """The oracle's Newton-Schulz statement (oracle.newton_schulz,
    gefen_muon.py:236-291: every product and elementwise result rounded to
    bf16) with fp32 GEMMs on the device (torch fp32 matmul on contiguous
    operands) instead of float64 on the host -- for shapes the host cannot
    run in seconds."""
    bf = lambda t: t.to(torch.bfloat16).float()
    x = bf(m)
    tall = x.shape[0] > x.shape[1]
    if tall:
        x = x.t().contiguous()
    norm = bf(torch.linalg.vector_norm(x.double()).float().reshape(1))
    norm = torch.clamp(norm, min=eps)
    x = bf(x / bf(norm))
    for a, b, c in sched:
        gram = bf(x @ x.t().contiguous())
        upd = bf(b * gram + c * (gram @ gram))
        x = bf(a * x + upd @ x)
    return x.t().contiguous() if tall else x


class StepTracker:
    """The reference's decomposed step (oracle.factored_step / block_step)
    for a set of parameters, started from the GPU optimizer's own step-1
    periods and codebook (each checked against the oracle's when it is
    learned), checked after every step: indices and magnitudes bit-exact,
    v_row / v_col / vmean within 1e-6, parameters within 1 ulp (fp32:
    1e-6 relative).  Parameters and grads are read in logical order, so
    transposed views and strided grads need nothing special."""

    def __init__(self, lr, wd, factored_2d, betas=(0.9, 0.999), eps=1e-8):
        self.lr, self.wd, self.factored_2d = lr, wd, factored_2d
        self.betas, self.eps = betas, eps
        self.ref = {}
        self.cb = None

    def track(self, name, p):
        self.ref[name] = {"p": _f(p).copy(), "dt": TDT_CODE[p.dtype], "shape": tuple(p.shape), "step": 0}

    def learn(self, opt, named, grads):
        """Step 1: the GPU's periods and codebook against the oracle's."""
        for name, p in named:
            r = self.ref[name]
            if "per" in r or name not in grads:
                continue
            per = int(opt.state[p]["automatic_period"])
            g = grads[name].reshape(-1)
            want = 1 if g.size == 1 else orc.find_period(g, r["shape"])
            assert per == want, "%s: period %d, oracle %d" % (name, per, want)
            r["per"] = per
        if self.cb is None:
            self.cb = orc.learn_codebook([(grads[n].reshape(-1), self.ref[n]["per"]) for n, _ in named
                                          if n in grads])
            np.testing.assert_array_equal(opt._gefen_codebook.cpu().numpy(), self.cb, err_msg="codebook")

    def step(self, name, g, lr=None):
        r = self.ref[name]
        lr = self.lr if lr is None else lr
        r["step"] += 1
        s = r["step"]
        bc1, bc2 = 1 - self.betas[0] ** s, 1 - self.betas[1] ** s
        per = r["per"]
        fact = self.factored_2d and len(r["shape"]) == 2
        if "idx" not in r:
            n = int(np.prod(r["shape"]))
            r["idx"], r["mag"] = np.zeros(n, np.uint8), np.zeros(n // per, np.float32)
            if fact:
                r["vr"], r["vc"] = np.zeros(r["shape"][0], np.float32), np.zeros(r["shape"][1], np.float32)
            else:
                r["vm"] = np.zeros(n // per, np.float32)
        kw = dict(beta1=self.betas[0], beta2=self.betas[1], lr=lr, eps=self.eps, bc1=bc1, bc2=bc2, wd=self.wd)
        if fact:
            r["p"], r["idx"], r["mag"], r["vr"], r["vc"] = orc.factored_step(
                r["p"], g, r["idx"], r["mag"], r["vr"], r["vc"], per, self.cb, r["dt"], **kw)
        else:
            r["p"], r["idx"], r["mag"], r["vm"] = orc.block_step(
                r["p"], g, r["idx"], r["mag"], r["vm"], per, self.cb, r["dt"], **kw)

    def check(self, opt, name, p, tag, lr=None):
        r = self.ref[name]
        st = opt.state[p]
        tag = "%s %s step %d" % (tag, name, r["step"])
        np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), r["idx"], err_msg=tag)
        np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), r["mag"], err_msg=tag)
        if "vr" in r:
            np.testing.assert_allclose(st["v_row"].cpu().numpy(), r["vr"], rtol=1e-6, err_msg=tag)
            np.testing.assert_allclose(st["v_col"].cpu().numpy(), r["vc"], rtol=1e-6, err_msg=tag)
        else:
            np.testing.assert_allclose(st["vmean"].cpu().numpy().reshape(-1), r["vm"], rtol=1e-6, err_msg=tag)
        got = _f(p).copy()
        assert_within_ulp(got, r["p"], r["dt"], tag, atol=1e-6 * (self.lr if lr is None else lr))
        r["p"] = got.reshape(r["shape"])  # continue from the GPU's parameters
