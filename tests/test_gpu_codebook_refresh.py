"""codebook_refresh_every on MI355X (reference gefen.py:3020-3070, 5743-5749):
every N steps the codebook is re-learned from the current grads with the
stored periods, and every stored index is mapped onto it through the nearest
rule applied to the old codeword it encodes; magnitudes stay.  Checked
against the oracle: the new codebook (histogram + exact DP) and the remapped
indices bit-exact, and the step that follows lands on oracle.factored_step /
block_step from the remapped state."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import assert_within_ulp

pytestmark = pytest.mark.gpu

LR, B1, B2, EPS, WD = 6e-5, 0.9, 0.999, 1e-8, 0.01


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _grads(gen, shapes, scale):
    return {n: (torch.randn(*s, generator=gen) * scale).to(torch.bfloat16) for n, s in shapes}


@pytest.mark.parametrize("factored", [True, False])
def test_refresh_matches_oracle(dev, factored):
    from gefen import Gefen
    gen = torch.Generator().manual_seed(17)
    shapes = [("w", (64, 96)), ("b", (96,))]
    ps = [(n, torch.nn.Parameter((torch.randn(*s, generator=gen) * 0.02).to(torch.bfloat16).to(dev)))
          for n, s in shapes]
    opt = Gefen(ps, lr=LR, betas=(B1, B2), eps=EPS, weight_decay=WD, factored_v_2d=factored,
                codebook_refresh_every=2)
    for _ in range(2):
        g = _grads(gen, shapes, 1e-3)
        for n, p in ps:
            p.grad = g[n].to(dev)
        opt.step()
    torch.cuda.synchronize()
    # step 3 re-learns first (global step 2 is a multiple of 2), then steps
    g3 = _grads(gen, shapes, 3e-3)  # another scale: the new codebook differs
    old_cb = opt._gefen_codebook.float().cpu().numpy()
    before = {}
    for n, p in ps:
        st = opt.state[p]
        before[n] = {"p": p.detach().float().cpu().numpy(), "idx": st["m_codebook"].cpu().numpy().reshape(-1),
                     "mag": st["m_magnitude"].cpu().numpy().reshape(-1), "period": int(st["automatic_period"]),
                     "step": int(st["step"])}
        if factored and p.ndim == 2:
            before[n].update(v_row=st["v_row"].cpu().numpy(), v_col=st["v_col"].cpu().numpy(),
                             fstep=int(st["factored_step"]))
        else:
            before[n].update(vmean=st["vmean"].cpu().numpy().reshape(-1), vstep=int(st["vmean_step"]))
    new_cb = orc.learn_codebook([(g3[n].float().numpy(), before[n]["period"]) for n, _ in shapes])
    for n, p in ps:
        p.grad = g3[n].to(dev)
    opt.step()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(opt._gefen_codebook.float().cpu().numpy(), new_cb, err_msg="re-learned codebook")
    assert not np.array_equal(new_cb, old_cb)
    for n, p in ps:
        b = before[n]
        st = opt.state[p]
        idx_re = orc.nearest_indices(new_cb, old_cb[b["idx"]])  # the remapped indices
        gf = g3[n].float().numpy()
        if factored and p.ndim == 2:
            s1, s2 = b["step"] + 1, b["fstep"] + 1
            p_ref, i_ref, m_ref, vr, vc = orc.factored_step(
                b["p"], gf, idx_re, b["mag"], b["v_row"], b["v_col"], b["period"], new_cb, orc.BF16, beta1=B1,
                beta2=B2, lr=LR, eps=EPS, bc1=1 - B1 ** s1, bc2=1 - B2 ** s2, wd=WD)
            np.testing.assert_allclose(st["v_row"].cpu().numpy(), vr, rtol=1e-6, err_msg=n)
            np.testing.assert_allclose(st["v_col"].cpu().numpy(), vc, rtol=1e-6, err_msg=n)
        else:
            s1, s2 = b["step"] + 1, b["vstep"] + 1
            p_ref, i_ref, m_ref, vm = orc.block_step(
                b["p"].reshape(-1), gf.reshape(-1), idx_re, b["mag"], b["vmean"], b["period"], new_cb, orc.BF16,
                beta1=B1, beta2=B2, lr=LR, eps=EPS, bc1=1 - B1 ** s1, bc2=1 - B2 ** s2, wd=WD)
            np.testing.assert_allclose(st["vmean"].cpu().numpy().reshape(-1), vm, rtol=1e-6, err_msg=n)
        np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), i_ref, err_msg=n + " indices")
        np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), m_ref, err_msg=n + " magnitudes")
        assert_within_ulp(p.detach().float().cpu().numpy().reshape(-1), np.asarray(p_ref).reshape(-1), orc.BF16,
                          n + " params", atol=1e-6 * LR)
