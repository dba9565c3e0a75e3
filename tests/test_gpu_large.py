"""BASELINE config 5 at full size: a 65536 x 40960 bf16 parameter (2,684,354,560
elements, factored) and a 1D bf16 parameter of 2^31 + 7 elements (block path,
period 1965 = the memory-safe fallback's largest divisor <= 2048, not a
multiple of 8, so the general kernels run), three plain Gefen steps through
the optimizer class.

The oracle cannot step 4.8e9 elements in seconds, so the checks use what is
local: a block's new indices and magnitude depend only on that block's grads,
indices and old magnitude (bit-exact against oracle.momentum_update / the
whole oracle block step for the 1D tensor); a row's v_row only on that row;
a column's v_col only on that column; an element's new value only on its own
inputs plus mean(v_row).  Samples sit at both ends and past element 2^31.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import assert_within_ulp

pytestmark = pytest.mark.gpu

R, C = 65536, 40960
N1 = (1 << 31) + 7
P2D = C          # one block per row
P1D = 1965
LR, BETAS, EPS, WD = 6e-5, (0.9, 0.999), 1e-8, 0.01


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    free, total = torch.cuda.mem_get_info(0)
    if free < 40 * (1 << 30):
        pytest.skip("needs about 40 GiB of free device memory")
    return torch.device("cuda", 0)


def _f(t):
    return t.detach().float().cpu().numpy()


def test_large_tensors_three_steps(dev):
    from gefen import Gefen
    import os
    cb_np = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "learn.npz"))["cb"]
    gen = torch.Generator(device=dev).manual_seed(0)
    w = torch.nn.Parameter(torch.empty(R, C, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=gen))
    b = torch.nn.Parameter(torch.empty(N1, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=gen))
    opt = Gefen([("w", w), ("b", b)], lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, factored_v_2d=True)
    opt._gefen_codebook = torch.from_numpy(cb_np).float().to(dev)
    opt.state[w]["automatic_period"] = P2D
    opt.state[b]["automatic_period"] = P1D
    rows = [0, 1, 52428, 52429, 60000, R - 1]                      # 52429 * C > 2^31
    cols = [0, 7, 20481, C - 1]
    nb1 = N1 // P1D
    blocks1 = [0, 1, nb1 // 2, nb1 - 3, nb1 - 2, nb1 - 1]             # the last block holds elements past 2^31
    assert (nb1 - 1) * P1D < (1 << 31) < nb1 * P1D
    for step in range(1, 4):
        w.grad = torch.empty_like(w).normal_(0.0, 1e-3, generator=gen)
        b.grad = torch.empty_like(b).normal_(0.0, 1e-3, generator=gen)
        sw = opt.state[w] if "step" in opt.state[w] else None
        sb = opt.state[b] if "step" in opt.state[b] else None
        # inputs of the sampled rows / columns / blocks before the step
        w_rows = _f(w[rows])
        g_rows = _f(w.grad[rows])
        g_cols = _f(w.grad[:, cols]).T
        idx_rows = sw["m_codebook"][rows].cpu().numpy() if sw else np.zeros((len(rows), C), np.uint8)
        mag_rows = sw["m_magnitude"][rows].cpu().numpy().reshape(-1) if sw else np.zeros(len(rows), np.float32)
        vr_old = sw["v_row"][rows].cpu().numpy() if sw else np.zeros(len(rows), np.float32)
        vc_old = sw["v_col"][cols].cpu().numpy() if sw else np.zeros(len(cols), np.float32)
        b_in = []
        for bk in blocks1:
            sl = slice(bk * P1D, (bk + 1) * P1D)
            b_in.append((_f(b[sl]), _f(b.grad[sl]),
                         sb["m_codebook"][bk].cpu().numpy() if sb else np.zeros(P1D, np.uint8),
                         sb["m_magnitude"][bk].cpu().numpy() if sb else np.zeros(1, np.float32),
                         sb["vmean"][bk].cpu().numpy() if sb else np.zeros(1, np.float32)))
        opt.step()
        torch.cuda.synchronize()
        sw, sb = opt.state[w], opt.state[b]
        bc1, bc2 = 1 - BETAS[0] ** step, 1 - BETAS[1] ** step
        # 1D: whole blocks through the oracle block step (bit-exact idx/mag)
        for bk, (p0, g0, i0, m0, v0) in zip(blocks1, b_in):
            p1, i1, m1, v1 = orc.block_step(p0, g0, i0, m0, v0, P1D, cb_np, orc.BF16, beta1=BETAS[0],
                                            beta2=BETAS[1], lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=WD)
            tag = "step %d 1D block %d" % (step, bk)
            np.testing.assert_array_equal(sb["m_codebook"][bk].cpu().numpy(), i1, err_msg=tag)
            np.testing.assert_array_equal(sb["m_magnitude"][bk].cpu().numpy(), m1, err_msg=tag)
            np.testing.assert_allclose(sb["vmean"][bk].cpu().numpy(), v1, rtol=1e-6, err_msg=tag)
            assert_within_ulp(_f(b[bk * P1D:(bk + 1) * P1D]), p1, orc.BF16, tag, atol=1e-6 * LR)
        # 2D: per-row momentum (one block per row), v_row / v_col, elements
        for j, r in enumerate(rows):
            i1, m1, q, _ = orc.momentum_update(g_rows[j], idx_rows[j], mag_rows[j:j + 1], P2D, cb_np, orc.BF16,
                                               BETAS[0])
            tag = "step %d row %d" % (step, r)
            np.testing.assert_array_equal(sw["m_codebook"][r].cpu().numpy(), i1, err_msg=tag + " indices")
            np.testing.assert_array_equal(sw["m_magnitude"][r].cpu().numpy(), m1, err_msg=tag + " magnitude")
            ms = np.float32(np.sum(g_rows[j].astype(np.float64) ** 2)) / np.float32(C)
            vr = np.float32(np.float64(ms) * np.float64(np.float32(1 - BETAS[1])) +
                            np.float64(np.float32(vr_old[j] * np.float32(BETAS[1]))))
            np.testing.assert_allclose(sw["v_row"][r].item(), vr, rtol=1e-6, err_msg=tag + " v_row")
        for j, c in enumerate(cols):
            ms = np.float32(np.sum(g_cols[j].astype(np.float64) ** 2)) / np.float32(R)
            vc = np.float32(np.float64(ms) * np.float64(np.float32(1 - BETAS[1])) +
                            np.float64(np.float32(vc_old[j] * np.float32(BETAS[1]))))
            np.testing.assert_allclose(sw["v_col"][c].item(), vc, rtol=1e-6, err_msg="step %d col %d" % (step, c))
        # elements of the sampled rows: the oracle's apply from the GPU's v
        v_row_all = sw["v_row"].cpu().numpy().astype(np.float64)
        mean = np.float32(np.sum(v_row_all) / R)
        v_col_all = sw["v_col"].cpu().numpy()
        for j, r in enumerate(rows):
            q = orc.round_dtype(cb_np[sw["m_codebook"][r].cpu().numpy()].astype(np.float32), orc.BF16) * \
                sw["m_magnitude"][r].item()
            vh = (np.float32(sw["v_row"][r].item()) * v_col_all) / mean
            h = np.sqrt(vh / np.float32(bc2)) + np.float32(EPS)
            stp = (np.float32(1.0) / h) * np.float32(1.0 / bc1)
            pw = orc.round_dtype((w_rows[j] * np.float32(1 - LR * WD)).astype(np.float32), orc.BF16)
            p_ref = orc.round_dtype((pw - (q * stp) * np.float32(LR)).astype(np.float32), orc.BF16)
            assert_within_ulp(_f(w[r]), p_ref, orc.BF16, "step %d row %d p" % (step, r), atol=1e-6 * LR)
