"""Parity of the HIP step (through the C ABI) with the CPU oracle and with the
reference's own golden trajectories.

Bar: requantized indices and block magnitudes bit-exact; parameters within
1 ulp of their dtype (fp32: 1e-6 relative); v_row / v_col / vmean within 1e-6
relative (the sums are taken in a different order than torch's CPU cascade).
"""
import os
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import assert_within_ulp

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
B1, B2, LR, EPS = 0.9, 0.999, 6e-5, 1e-8
TDT = {orc.F32: torch.float32, orc.F16: torch.float16, orc.BF16: torch.bfloat16}
P_RTOL = {orc.F32: 1e-6, orc.F16: 2.0 ** -10, orc.BF16: 2.0 ** -7}


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from gefen.kernels import _native
    _native.load()
    return torch.device("cuda", 0)


def _codebook():
    return np.load(os.path.join(GOLD, "learn.npz"))["cb"]


def _assert_p(got, ref, dtype, msg):
    """fp32: 1e-6 relative per element (the fp32 step rounds in the
    reference's op order); half types: 1 ulp of the reference value in its
    dtype (the exact spacing of its binade) plus 1e-6 * lr absolute -- the
    16-bit factored stepsize is sqrt(v_row*s) * sqrt(v_col), ulps off the
    reference's rounding, which is what remains visible where p itself
    cancels towards zero."""
    assert_within_ulp(got, ref, dtype, msg, atol=1e-6 * LR)


def _run_factored(dev, dtype, rows, cols, period, wd, steps, seed, transposed=False, sr_seed=None):
    from gefen.kernels import automatic_gefen_fused as fused
    gen = torch.Generator().manual_seed(seed)
    tdt = TDT[dtype]
    cb = _codebook()
    cb_dev = torch.from_numpy(cb).to(dev)
    p0 = (torch.randn(rows, cols, generator=gen) * 0.02).to(tdt)
    if transposed:
        storage = p0.t().contiguous().to(dev)  # [cols, rows]
        p_dev = storage.t()                    # logical [rows, cols], strides (1, rows)
    else:
        p_dev = p0.to(dev)
    nb = rows * cols // period
    idx = torch.zeros(nb, period, dtype=torch.uint8, device=dev)
    mag = torch.zeros(nb, 1, dtype=torch.float32, device=dev)
    vr = torch.zeros(rows, dtype=torch.float32, device=dev)
    vc = torch.zeros(cols, dtype=torch.float32, device=dev)
    st = {"p": p0.float().numpy(), "idx": np.zeros(rows * cols, np.uint8),
          "mag": np.zeros(nb, np.float32), "v_row": np.zeros(rows, np.float32),
          "v_col": np.zeros(cols, np.float32)}
    for s in range(1, steps + 1):
        g = (torch.randn(rows, cols, generator=gen) * 10 ** gen_uniform(gen, -4, -2)).to(tdt)
        bc1, bc2 = 1 - B1 ** s, 1 - B2 ** s
        seed_s = None if sr_seed is None else sr_seed + s
        fused.gefen_factored_update_cuda(
            p_dev, g.to(dev).reshape(-1).view(nb, period), idx, mag, vr, vc, cb_dev, cols,
            B1, B2, LR, EPS, 1.0 / bc2, 1.0 / bc1, 1.0 - LR * wd,
            stochastic_round=seed_s is not None, rng_seed=seed_s or 0)
        p_np, i_np, m_np, r_np, c_np = orc.factored_step(
            st["p"], g.float().numpy(), st["idx"], st["mag"], st["v_row"], st["v_col"], period,
            cb, dtype, beta1=B1, beta2=B2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=wd, sr_seed=seed_s)
        torch.cuda.synchronize()
        tag = "factored %s [%d,%d] P=%d wd=%g step %d%s%s" % (tdt, rows, cols, period, wd, s,
                                                              " transposed" if transposed else "",
                                                              "" if seed_s is None else " sr seed %d" % seed_s)
        np.testing.assert_array_equal(idx.cpu().numpy().reshape(-1), i_np, err_msg=tag + " idx")
        np.testing.assert_array_equal(mag.cpu().numpy().reshape(-1), m_np, err_msg=tag + " mag")
        np.testing.assert_allclose(vr.cpu().numpy(), r_np, rtol=1e-6, err_msg=tag + " v_row")
        np.testing.assert_allclose(vc.cpu().numpy(), c_np, rtol=1e-6, err_msg=tag + " v_col")
        _assert_p(p_dev.float().cpu().numpy(), p_np, dtype, tag + " p")
        # continue from the GPU state so sums never drift apart
        st = {"p": p_dev.float().cpu().numpy(), "idx": i_np, "mag": m_np,
              "v_row": vr.cpu().numpy(), "v_col": vc.cpu().numpy()}
    return tag


def gen_uniform(gen, lo, hi):
    return float(torch.rand(1, generator=gen)) * (hi - lo) + lo


FACTORED_CASES = [
    (orc.BF16, 64, 96, 768, 0.01),
    (orc.BF16, 64, 96, 3072, 0.0),
    (orc.BF16, 48, 128, 16, 0.01),
    (orc.F32, 64, 96, 96, 0.01),
    (orc.F32, 40, 72, 1440, 0.01),
    (orc.F16, 32, 64, 64, 0.01),
    (orc.BF16, 30, 50, 3, 0.01),      # cols % 8 != 0, tiny period: generic path
    (orc.BF16, 7, 4100, 28700, 0.01),  # 2 column tiles, ragged tail
    (orc.F32, 300, 24, 1, 0.0),        # period 1: one block per element
    (orc.BF16, 1024, 2048, 1 << 20, 0.01),
    # row-segment apply (512-column segments of 8 rows): a short last
    # segment and a 4-row last tile; block boundaries inside segments (fp32);
    # whole segments; one segment per row and a 1-row last tile
    (orc.BF16, 100, 1000, 800, 0.01),
    (orc.F32, 96, 1024, 768, 0.01),
    (orc.BF16, 24, 2560, 20480, 0.0),
    (orc.F16, 17, 512, 4352, 0.01),
]


@pytest.mark.parametrize("case", FACTORED_CASES, ids=lambda c: "%s-%dx%d-P%d-wd%g" % c)
def test_factored_matches_oracle(dev, case):
    dtype, rows, cols, period, wd = case
    _say("case", _run_factored(dev, dtype, rows, cols, period, wd, 3, seed=rows * 7 + cols))


NONFINITE_CASES = ["nan", "inf", "huge", "tiny_mag"]


@pytest.mark.parametrize("kind", NONFINITE_CASES)
def test_factored_nonfinite_grads_block_max(dev, kind):
    """Block magnitudes and indices when grads hold NaN, inf, values whose
    square overflows fp32 (1e20), or when the old magnitude is huge.  The
    stats pass takes the |u| max as floats only while every u is provably
    finite and falls back to the ordered-integer max (NaN above inf, torch's
    amax) otherwise; both must give the oracle's magnitudes bit for bit."""
    from gefen.kernels import automatic_gefen_fused as fused
    rows, cols, period = 64, 1024, 8192  # full column tiles, 8 rows per block
    gen = torch.Generator().manual_seed(17)
    cb = _codebook()
    cb_dev = torch.from_numpy(cb).to(dev)
    p0 = (torch.randn(rows, cols, generator=gen) * 0.02).to(torch.bfloat16)
    p_dev = p0.to(dev)
    nb = rows * cols // period
    idx = torch.zeros(nb, period, dtype=torch.uint8, device=dev)
    mag = torch.zeros(nb, 1, dtype=torch.float32, device=dev)
    vr = torch.zeros(rows, dtype=torch.float32, device=dev)
    vc = torch.zeros(cols, dtype=torch.float32, device=dev)
    st = {"p": p0.float().numpy(), "idx": np.zeros(rows * cols, np.uint8), "mag": np.zeros(nb, np.float32),
          "v_row": np.zeros(rows, np.float32), "v_col": np.zeros(cols, np.float32)}
    for s in range(1, 4):
        g = torch.randn(rows, cols, generator=gen) * 1e-3
        if s >= 2:  # step 1 builds finite state; later steps plant the values
            if kind == "nan":
                g[3, 100] = float("nan")      # block 0
                g[40, 1000] = float("nan")    # block 5
            elif kind == "inf":
                g[9, 7] = float("inf")        # block 1
                g[20, 512] = float("-inf")    # block 2
            elif kind == "huge":
                g[12, 300] = 1e20             # g^2 overflows fp32: exact fallback
                g[50, 900] = -3e19
        g = g.to(torch.bfloat16)
        if kind == "tiny_mag" and s == 2:
            # huge old magnitudes (>= 1e38) must take the exact path
            m_host = torch.from_numpy(st["mag"]).clone()
            m_host[3] = 2e38
            m_host[6] = 3.0e38
            mag.copy_(m_host.view(nb, 1))
            st["mag"] = m_host.numpy()
        bc1, bc2 = 1 - B1 ** s, 1 - B2 ** s
        fused.gefen_factored_update_cuda(
            p_dev, g.to(dev).reshape(-1).view(nb, period), idx, mag, vr, vc, cb_dev, cols,
            B1, B2, LR, EPS, 1.0 / bc2, 1.0 / bc1, 1.0 - LR * 0.01)
        p_np, i_np, m_np, r_np, c_np = orc.factored_step(
            st["p"], g.float().numpy(), st["idx"], st["mag"], st["v_row"], st["v_col"], period,
            cb, orc.BF16, beta1=B1, beta2=B2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=0.01)
        torch.cuda.synchronize()
        tag = "nonfinite %s step %d" % (kind, s)
        _say(tag)
        np.testing.assert_array_equal(mag.cpu().numpy().reshape(-1), m_np, err_msg=tag + " mag")
        np.testing.assert_array_equal(idx.cpu().numpy().reshape(-1), i_np, err_msg=tag + " idx")
        st = {"p": p_dev.float().cpu().numpy(), "idx": i_np, "mag": m_np,
              "v_row": vr.cpu().numpy(), "v_col": vc.cpu().numpy()}


@pytest.mark.parametrize("dtype", [orc.BF16, orc.F32])
def test_factored_transposed_view_matches_oracle(dev, dtype):
    _say("case", _run_factored(dev, dtype, 96, 64, 768, 0.01, 2, seed=5, transposed=True))


def _strided(t2d, layout, dev, pad=16):
    """Device copy of a logical [R, C] tensor in the given storage layout:
    'contig' row-major; 'view' the .t() of a contiguous [C, R] tensor (strides
    (1, R)); 'view_ld' the same with storage rows of R + pad (strides
    (1, R + pad))."""
    if layout == "contig":
        return t2d.contiguous().to(dev)
    if layout == "view":
        return t2d.t().contiguous().to(dev).t()
    R, C = t2d.shape
    st = torch.zeros(C, R + pad, dtype=t2d.dtype)
    st[:, :R] = t2d.t()
    return st.to(dev)[:, :R].t()


def _run_factored_strided(dev, dtype, rows, cols, period, p_layout, g_layout, steps=3, seed=0, wd=0.01):
    """gefenx_factored_update through the C ABI with the parameter and the
    grad in the given storage layouts (their strides go to the kernel as is)
    against the oracle's logical row-major step."""
    from gefen.kernels import _native
    from gefen.kernels import automatic_gefen_fused as fused
    lib = _native.load()
    gen = torch.Generator().manual_seed(seed)
    tdt = TDT[dtype]
    cb = _codebook()
    cb_dev = torch.from_numpy(cb).to(dev)
    qt = fused.quant_table(cb_dev, tdt)
    p0 = (torch.randn(rows, cols, generator=gen) * 0.02).to(tdt)
    p_dev = _strided(p0, p_layout, dev)
    nb = rows * cols // period
    idx = torch.zeros(nb, period, dtype=torch.uint8, device=dev)
    mag = torch.zeros(nb, 1, dtype=torch.float32, device=dev)
    vr = torch.zeros(rows, dtype=torch.float32, device=dev)
    vc = torch.zeros(cols, dtype=torch.float32, device=dev)
    ws = torch.zeros(int(lib.gefenx_workspace_bytes(_native.WS_FACTORED, rows, cols, nb)), dtype=torch.uint8,
                     device=dev)
    st = {"p": p0.float().numpy(), "idx": np.zeros(rows * cols, np.uint8), "mag": np.zeros(nb, np.float32),
          "v_row": np.zeros(rows, np.float32), "v_col": np.zeros(cols, np.float32)}
    tag = ""
    for s in range(1, steps + 1):
        g = (torch.randn(rows, cols, generator=gen) * 10 ** gen_uniform(gen, -4, -2)).to(tdt)
        g_dev = _strided(g, g_layout, dev)
        bc1, bc2 = 1 - B1 ** s, 1 - B2 ** s
        tag = "factored %s [%d,%d] P=%d p:%s g:%s step %d" % (tdt, rows, cols, period, p_layout, g_layout, s)
        _say("case", tag)
        _native.check(lib.gefenx_factored_update(
            p_dev.data_ptr(), g_dev.data_ptr(), fused._dtype_code(tdt), rows, cols,
            p_dev.stride(0), p_dev.stride(1), g_dev.stride(0), g_dev.stride(1),
            idx.data_ptr(), mag.data_ptr(), vr.data_ptr(), vc.data_ptr(), period, qt.data_ptr(),
            B1, B2, LR, EPS, 1.0 / bc2, 1.0 / bc1, 1.0 - LR * wd, 0, 0, None, None,
            ws.data_ptr(), ws.numel(), torch.cuda.current_stream(dev).cuda_stream), tag)
        p_np, i_np, m_np, r_np, c_np = orc.factored_step(
            st["p"], g.float().numpy(), st["idx"], st["mag"], st["v_row"], st["v_col"], period,
            cb, dtype, beta1=B1, beta2=B2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=wd)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(idx.cpu().numpy().reshape(-1), i_np, err_msg=tag + " idx")
        np.testing.assert_array_equal(mag.cpu().numpy().reshape(-1), m_np, err_msg=tag + " mag")
        np.testing.assert_allclose(vr.cpu().numpy(), r_np, rtol=1e-6, err_msg=tag + " v_row")
        np.testing.assert_allclose(vc.cpu().numpy(), c_np, rtol=1e-6, err_msg=tag + " v_col")
        _assert_p(p_dev.float().cpu().numpy(), p_np, dtype, tag + " p")
        st = {"p": p_dev.float().cpu().numpy(), "idx": i_np, "mag": m_np,
              "v_row": vr.cpu().numpy(), "v_col": vc.cpu().numpy()}
    return tag


# Transposed-view kernels (strides (1, ld)): ragged 64-tiles, blocks that
# straddle rows, several 1024-column tiles and 64-row bands per workgroup,
# one-chunk blocks (P = 8) and a single block.
STRIDED_CASES = [
    (orc.BF16, 200, 136, 400, "view", "view"),
    (orc.BF16, 200, 136, 400, "view_ld", "view_ld"),
    (orc.BF16, 4104, 4120, 1080, "view", "view"),
    (orc.F32, 328, 200, 1640, "view", "view"),
    (orc.F16, 136, 264, 88, "view_ld", "view"),
    (orc.BF16, 64, 64, 8, "view", "view"),
    (orc.BF16, 128, 192, 24576, "view", "view"),
    # R and C multiples of 64: workgroups of four interior tiles take the
    # full-tile apply (unconditional loads and stores), the last the general one
    (orc.F32, 256, 192, 512, "view", "view"),
    (orc.F16, 128, 384, 192, "view_ld", "view"),
    (orc.BF16, 200, 136, 400, "contig", "view"),    # view stats, general apply
    (orc.F32, 200, 136, 400, "view", "contig"),      # contiguous stats, general apply
    # periods above 21 * (C + 1): every 64 x 64 tile touches at most 4
    # blocks (scalar block loads), with block edges inside rows
    (orc.BF16, 512, 320, 8192, "view", "view"),
    (orc.F32, 256, 384, 12288, "view", "view"),
    (orc.F16, 448, 200, 5600, "view_ld", "view_ld"),
]


@pytest.mark.parametrize("case", STRIDED_CASES, ids=lambda c: "%s-%dx%d-P%d-p_%s-g_%s" % c)
def test_factored_strided_matches_oracle(dev, case):
    dtype, rows, cols, period, pl, gl = case
    _run_factored_strided(dev, dtype, rows, cols, period, pl, gl, seed=rows + cols)


BLOCK_VIEW_CASES = [
    (orc.BF16, 200, 136, 400, "view"),
    (orc.BF16, 200, 136, 400, "view_ld"),
    (orc.F32, 328, 200, 1640, "view"),
    (orc.F16, 136, 264, 88, "view"),
    (orc.BF16, 1096, 2056, 2056, "view"),
    (orc.BF16, 320, 256, 640, "view"),  # full-tile apply workgroups and a partial last one
    (orc.F32, 256, 128, 64, "view_ld"),
    (orc.BF16, 512, 320, 8192, "view"),  # at most 4 blocks per 64 x 64 tile
    (orc.F16, 448, 200, 5600, "view_ld"),
]


@pytest.mark.parametrize("case", BLOCK_VIEW_CASES, ids=lambda c: "%s-%dx%d-P%d-%s" % c)
def test_block_view_matches_oracle(dev, case):
    """factored_v_2d=False with a transposed-view parameter and grad: the
    multi-tensor launcher steps it in place (tiled view kernels, block
    vmean) -- indices and magnitudes bit-exact against the oracle's block
    step, vmean within 1e-6, params within 1 ulp."""
    from gefen import Gefen
    dtype, rows, cols, period, layout = case
    gen = torch.Generator().manual_seed(rows * 3 + cols)
    tdt = TDT[dtype]
    cb = _codebook()
    p0 = (torch.randn(rows, cols, generator=gen) * 0.02).to(tdt)
    p = torch.nn.Parameter(_strided(p0, layout, dev))
    assert p.stride(0) == 1
    wd = 0.01
    opt = Gefen([("w", p)], lr=LR, betas=(B1, B2), eps=EPS, weight_decay=wd, factored_v_2d=False)
    opt._gefen_codebook = torch.from_numpy(cb).float().to(dev)
    opt.state[p]["automatic_period"] = period
    nb = rows * cols // period
    ref = {"p": p0.float().numpy(), "idx": np.zeros(rows * cols, np.uint8), "mag": np.zeros(nb, np.float32),
           "vm": np.zeros(nb, np.float32)}
    for s in range(1, 4):
        g = (torch.randn(rows, cols, generator=gen) * 10 ** gen_uniform(gen, -4, -2)).to(tdt)
        p.grad = _strided(g, layout, dev)
        tag = "block view %s [%d,%d] P=%d %s step %d" % (tdt, rows, cols, period, layout, s)
        _say("case", tag)
        opt.step()
        torch.cuda.synchronize()
        bc1, bc2 = 1 - B1 ** s, 1 - B2 ** s
        p1, i1, m1, v1 = orc.block_step(ref["p"], g.float().numpy(), ref["idx"], ref["mag"], ref["vm"], period,
                                        cb, dtype, beta1=B1, beta2=B2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=wd)
        st = opt.state[p]
        np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), i1, err_msg=tag + " idx")
        np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), m1, err_msg=tag + " mag")
        np.testing.assert_allclose(st["vmean"].cpu().numpy().reshape(-1), v1, rtol=1e-6, err_msg=tag + " vmean")
        _assert_p(p.detach().float().cpu().numpy(), p1, dtype, tag + " p")
        ref = {"p": p.detach().float().cpu().numpy(), "idx": i1, "mag": m1, "vm": st["vmean"].cpu().numpy().reshape(-1)}


def _run_block(dev, dtype, n, period, wd, steps, seed, sr_seed=None):
    from gefen.kernels import automatic_gefen_fused as fused
    gen = torch.Generator().manual_seed(seed)
    tdt = TDT[dtype]
    cb = _codebook()
    cb_dev = torch.from_numpy(cb).to(dev)
    p0 = (torch.randn(n, generator=gen) * 0.02).to(tdt)
    p_dev = p0.to(dev)
    nb = n // period
    idx = torch.zeros(nb, period, dtype=torch.uint8, device=dev)
    mag = torch.zeros(nb, 1, dtype=torch.float32, device=dev)
    vm = torch.zeros(nb, 1, dtype=torch.float32, device=dev)
    st = {"p": p0.float().numpy(), "idx": np.zeros(n, np.uint8), "mag": np.zeros(nb, np.float32),
          "vmean": np.zeros(nb, np.float32)}
    for s in range(1, steps + 1):
        g = (torch.randn(n, generator=gen) * 1e-3).to(tdt)
        bc1, bc2 = 1 - B1 ** s, 1 - B2 ** s
        seed_s = None if sr_seed is None else sr_seed + s
        fused.automatic_gefen_fused_full_update_cuda(
            p_dev, g.to(dev).view(nb, period), idx, mag, vm, cb_dev, False, B1, B2, LR, EPS,
            1.0 / np.sqrt(bc2), 1.0 / bc1, 1.0 - LR * wd,
            stochastic_round=seed_s is not None, rng_seed=seed_s or 0)
        p_np, i_np, m_np, v_np = orc.block_step(
            st["p"], g.float().numpy(), st["idx"], st["mag"], st["vmean"], period, cb, dtype,
            beta1=B1, beta2=B2, lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=wd, sr_seed=seed_s)
        torch.cuda.synchronize()
        tag = "block %s n=%d P=%d wd=%g step %d%s" % (tdt, n, period, wd, s,
                                                     "" if seed_s is None else " sr seed %d" % seed_s)
        np.testing.assert_array_equal(idx.cpu().numpy().reshape(-1), i_np, err_msg=tag + " idx")
        np.testing.assert_array_equal(mag.cpu().numpy().reshape(-1), m_np, err_msg=tag + " mag")
        np.testing.assert_allclose(vm.cpu().numpy().reshape(-1), v_np, rtol=1e-6, err_msg=tag + " vmean")
        _assert_p(p_dev.float().cpu().numpy(), p_np, dtype, tag + " p")
        st = {"p": p_dev.float().cpu().numpy(), "idx": i_np, "mag": m_np,
              "vmean": vm.cpu().numpy().reshape(-1)}
    return tag


BLOCK_CASES = [
    (orc.BF16, 4096, 4096, 0.01),
    (orc.BF16, 4096, 64, 0.0),
    (orc.BF16, 4096, 1, 0.01),
    (orc.F32, 1000, 8, 0.01),
    (orc.F32, 999, 27, 0.0),
    (orc.F16, 3000, 24, 0.01),
    (orc.BF16, 1 << 20, 1 << 19, 0.01),
    (orc.BF16, 7, 7, 0.01),
    (orc.BF16, 122880, 24576, 0.01),   # blocks straddle stats workgroups at odd offsets
    (orc.F32, 122880, 40, 0.01),       # several blocks per wave
    (orc.F16, 99999, 11111, 0.01),     # P % 8 != 0: one element per item, blocks over ~5 workgroups
    (orc.BF16, 3 << 22, 3 << 21, 0.01),  # two blocks of 768 stats workgroups each (workgroup-wide finalize)
]


@pytest.mark.parametrize("case", BLOCK_CASES, ids=lambda c: "%s-n%d-P%d-wd%g" % c)
def test_block_matches_oracle(dev, case):
    dtype, n, period, wd = case
    _say("case", _run_block(dev, dtype, n, period, wd, 3, seed=n + period))


SR_FACTORED_CASES = [
    (orc.BF16, 64, 96, 768, False),
    (orc.F32, 40, 72, 1440, False),
    (orc.BF16, 30, 50, 3, False),       # generic path
    (orc.BF16, 96, 64, 768, True),      # transposed view: logical element index
    (orc.BF16, 1024, 2048, 1 << 20, False),
]


@pytest.mark.parametrize("case", SR_FACTORED_CASES, ids=lambda c: "%s-%dx%d-P%d-T%d" % c)
def test_factored_stochastic_rounding_matches_oracle(dev, case):
    """stochastic_round=True: the HIP kernels' SplitMix64 rounding against
    oracle.factored_step(sr_seed=...) index for index (seed 2^40 + step, so
    the seed's high bits are exercised)."""
    dtype, rows, cols, period, transposed = case
    _say("case", _run_factored(dev, dtype, rows, cols, period, 0.01, 3, seed=rows + cols, transposed=transposed,
                               sr_seed=(1 << 40)))


@pytest.mark.parametrize("case", [(orc.BF16, 4096, 64), (orc.F32, 999, 27), (orc.BF16, 1 << 20, 1 << 19)],
                         ids=lambda c: "%s-n%d-P%d" % c)
def test_block_stochastic_rounding_matches_oracle(dev, case):
    dtype, n, period = case
    _say("case", _run_block(dev, dtype, n, period, 0.01, 3, seed=n, sr_seed=12345))


GOLDEN_CASES = ["fact_f32", "fact_bf16", "fact_f16", "block_bf16", "block_f32", "block_f16",
                "zeros_f32"]
NAME_DT = {"f32": orc.F32, "bf16": orc.BF16, "f16": orc.F16}


@pytest.mark.parametrize("name", GOLDEN_CASES)
def test_reference_golden_trajectory_on_gpu(dev, name):
    """Replay the reference's CPU trajectory through the HIP kernels: at every
    step start from the reference's state and compare with its next state."""
    from gefen.kernels import automatic_gefen_fused as fused
    z = np.load(os.path.join(GOLD, "step_%s.npz" % name))
    dtype = NAME_DT[name.split("_")[1]]
    tdt = TDT[dtype]
    cb_dev = torch.from_numpy(z["codebook"]).to(dev)
    wd = float(z["wd"])
    pnames = sorted({k.split("_", 1)[1] for k in z.files if k.startswith("p0_")})
    for pn in pnames:
        p0 = z["p0_" + pn]
        per = int(z["period_" + pn])
        nb = p0.size // per
        factored = bool(int(z["factored"])) and p0.ndim == 2
        prev = {"p": p0, "idx": np.zeros(p0.size, np.uint8), "mag": np.zeros(nb, np.float32),
                "v_row": np.zeros(p0.shape[0], np.float32) if factored else None,
                "v_col": np.zeros(p0.shape[-1], np.float32) if factored else None,
                "vmean": None if factored else np.zeros(nb, np.float32)}
        for s in range(1, int(z["steps"]) + 1):
            bc1, bc2 = 1 - B1 ** s, 1 - B2 ** s
            p_dev = torch.from_numpy(np.ascontiguousarray(prev["p"])).to(tdt).to(dev)
            g_dev = torch.from_numpy(z["g%d_%s" % (s, pn)]).to(tdt).to(dev).reshape(-1).view(nb, per)
            idx = torch.from_numpy(np.ascontiguousarray(prev["idx"]).reshape(nb, per)).to(dev)
            mag = torch.from_numpy(np.ascontiguousarray(prev["mag"]).reshape(nb, 1)).to(dev)
            tag = "%s/%s step %d" % (name, pn, s)
            if factored:
                vr = torch.from_numpy(np.ascontiguousarray(prev["v_row"])).to(dev)
                vc = torch.from_numpy(np.ascontiguousarray(prev["v_col"])).to(dev)
                fused.gefen_factored_update_cuda(p_dev, g_dev, idx, mag, vr, vc, cb_dev, p0.shape[1],
                                                 B1, B2, LR, EPS, 1.0 / bc2, 1.0 / bc1, 1.0 - LR * wd)
            else:
                vm = torch.from_numpy(np.ascontiguousarray(prev["vmean"]).reshape(nb, 1)).to(dev)
                fused.automatic_gefen_fused_full_update_cuda(
                    p_dev, g_dev, idx, mag, vm, cb_dev, False, B1, B2, LR, EPS,
                    1.0 / np.sqrt(bc2), 1.0 / bc1, 1.0 - LR * wd)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(idx.cpu().numpy().reshape(-1), z["idx%d_%s" % (s, pn)],
                                          err_msg=tag + " idx")
            np.testing.assert_array_equal(mag.cpu().numpy().reshape(-1), z["mag%d_%s" % (s, pn)],
                                          err_msg=tag + " mag")
            _assert_p(p_dev.float().cpu().numpy(), z["p%d_%s" % (s, pn)], dtype, tag + " p")
            if factored:
                np.testing.assert_allclose(vr.cpu().numpy(), z["v_row%d_%s" % (s, pn)], rtol=1e-6)
                np.testing.assert_allclose(vc.cpu().numpy(), z["v_col%d_%s" % (s, pn)], rtol=1e-6)
            else:
                np.testing.assert_allclose(vm.cpu().numpy().reshape(-1), z["vmean%d_%s" % (s, pn)],
                                           rtol=1e-6)
            prev = {"p": z["p%d_%s" % (s, pn)].reshape(p0.shape), "idx": z["idx%d_%s" % (s, pn)],
                    "mag": z["mag%d_%s" % (s, pn)],
                    "v_row": z["v_row%d_%s" % (s, pn)] if factored else None,
                    "v_col": z["v_col%d_%s" % (s, pn)] if factored else None,
                    "vmean": None if factored else z["vmean%d_%s" % (s, pn)]}
        _say("case golden", name, pn, "ok")


