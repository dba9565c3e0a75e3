"""GPU parity of the Muon kernels against the oracle (through the C ABI).

- the bf16 MFMA GEMM behind Newton-Schulz against a float64 product rounded
  to bf16 (odd shapes, K not a multiple of 8, alpha/beta epilogue);
- the quantised Muon momentum: indices, magnitudes and the emitted momentum
  bit-exact against oracle.muon_momentum (bf16 / fp16 / fp32, Nesterov on/off);
- Newton-Schulz against oracle.newton_schulz and the reference's own outputs;
- NorMuon scale and the Muon apply against the oracle.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TORCH_DT = {orc.F32: torch.float32, orc.F16: torch.float16, orc.BF16: torch.bfloat16}
NS_REL = 2e-2  # the reference's own batched-vs-serial Newton-Schulz bound


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


@pytest.fixture(scope="module")
def lib():
    from gefen.kernels import _native
    return _native.load()


def _check(rc, lib):
    from gefen.kernels import _native
    _native.check(rc, "call")


def _stream(dev):
    return torch.cuda.current_stream(dev).cuda_stream


def _bf16_np(t):
    return t.float().cpu().numpy()


# K % 64 == 0 with 16-byte aligned operands takes a direct-to-LDS kernel:
# 128 x 128 tiles for (256, 192, 128), (200, 136, 192), (130, 300, 64) (full
# tiles, partial tiles, a single K step), 256 x 256 tiles once those fill the
# CUs (the last three: full tiles on the 16x16x32 kernel, partial edge tiles
# on the 32x32x16 one, a single K step on the 16x16x32 one); the rest the
# register-staged one (K = 30 also without 16-byte loads)
@pytest.mark.parametrize("mnk", [(128, 128, 32), (256, 192, 160), (200, 136, 72), (100, 60, 30), (33, 257, 48),
                                 (256, 192, 128), (200, 136, 192), (130, 300, 64),
                                 (4096, 4096, 128), (4000, 4200, 192), (4096, 4096, 64)])
def test_gemm_nt_matches_float64(dev, lib, mnk):
    M, N, K = mnk
    gen = torch.Generator(device="cpu").manual_seed(M * 7 + N + K)
    A = torch.randn(M, K, generator=gen).to(torch.bfloat16)
    B = torch.randn(N, K, generator=gen).to(torch.bfloat16)
    C = torch.randn(M, N, generator=gen).to(torch.bfloat16)
    for alpha, beta, use_c in ((1.0, 0.0, False), (0.75, -1.5, True)):
        Ad, Bd, Cd = A.to(dev), B.to(dev), C.to(dev)
        D = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        _check(lib.gefenx_gemm_nt_bf16(Ad.data_ptr(), Bd.data_ptr(), Cd.data_ptr() if use_c else None, D.data_ptr(),
                                       M, N, K, alpha, beta, _stream(dev)), lib)
        torch.cuda.synchronize()
        ref = alpha * (A.double() @ B.double().T)
        if use_c:
            ref = ref + beta * C.double()
        ref_b = orc.bf16(ref.numpy().astype(np.float32))
        got = _bf16_np(D)
        # fp32 accumulation in another order than float64: an element may
        # round to the neighbouring bf16 value
        assert np.mean(got == ref_b) > 0.98, "gemm %s alpha %g: exact %.4f" % (mnk, alpha, np.mean(got == ref_b))
        np.testing.assert_allclose(got, ref_b, rtol=2.0 ** -7, atol=2.0 ** -7 * np.abs(ref_b).max() * 2 ** -6)


def _mom_state(numel, period, seed):
    rng = np.random.default_rng(seed)
    idx = rng.integers(0, 256, numel).astype(np.uint8)
    mag = (rng.random(numel // period) * 1e-3).astype(np.float32)
    return idx, mag


MOM_CASES = [(orc.BF16, 96 * 40, 96, True), (orc.BF16, 4096, 512, False), (orc.F32, 3000, 24, True),
             (orc.F16, 2048, 64, True), (orc.BF16, 1000, 1000, True), (orc.BF16, 999, 27, False)]


@pytest.mark.parametrize("case", MOM_CASES, ids=lambda c: "dt%d-n%d-P%d-nest%d" % c)
def test_muon_momentum_matches_oracle(dev, lib, case):
    dtype, numel, period, nesterov = case
    from gefen.kernels import _native
    from gefen.kernels import automatic_gefen_fused as fused
    td = TORCH_DT[dtype]
    rng = np.random.default_rng(numel + period)
    cb = np.load(os.path.join(GOLDEN, "learn.npz"))["cb"].astype(np.float32)
    qt = fused.quant_table(torch.from_numpy(cb).to(dev), td)
    idx_np, mag_np = _mom_state(numel, period, 1)
    idx = torch.from_numpy(idx_np.copy()).to(dev)
    mag = torch.from_numpy(mag_np.copy()).to(dev)
    ws = torch.zeros(int(lib.gefenx_workspace_bytes(_native.WS_MOMENTUM, 0, 0, numel // period)) + 256,
                     dtype=torch.uint8, device=dev)
    for step in range(3):
        g = torch.from_numpy((rng.standard_normal(numel) * 1e-3).astype(np.float32)).to(td)
        if step == 1 and numel >= 2 * period:
            g[:period] = 0  # a block whose magnitude decays towards zero
        out = torch.empty(numel, dtype=td, device=dev)
        gd = g.to(dev)
        _check(lib.gefenx_quantized_momentum_update(gd.data_ptr(), fused._dtype_code(td), numel, period,
                                                    idx.data_ptr(), mag.data_ptr(), qt.data_ptr(), out.data_ptr(),
                                                    0.95, 0, 0, None, 1 if nesterov else 0, ws.data_ptr(),
                                                    ws.numel(), _stream(dev)), lib)
        torch.cuda.synchronize()
        idx_np, mag_np, out_np = orc.muon_momentum(g.float().numpy(), idx_np, mag_np, period, cb, dtype, 0.95,
                                                   nesterov)
        tag = "step %d %s" % (step, case)
        np.testing.assert_array_equal(idx.cpu().numpy(), idx_np, err_msg=tag + " indices")
        np.testing.assert_array_equal(mag.cpu().numpy(), mag_np, err_msg=tag + " magnitudes")
        np.testing.assert_array_equal(out.float().cpu().numpy(), out_np, err_msg=tag + " momentum")


def _ns_gpu(dev, lib, m, sched, in_dtype=torch.bfloat16):
    from gefen.kernels import automatic_gefen_fused as fused
    x = torch.from_numpy(np.asarray(m, np.float32)).to(in_dtype).to(dev)
    if x.dim() == 2:
        x = x.unsqueeze(0)
    b, r, c = x.shape
    out = torch.empty(b, r, c, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(int(lib.gefenx_ns_workspace_bytes(b, r, c)), dtype=torch.uint8, device=dev)
    abc = np.ascontiguousarray(np.asarray(sched, np.float64).reshape(-1))
    _check(lib.gefenx_newton_schulz(x.data_ptr(), fused._dtype_code(in_dtype), out.data_ptr(), b, r, c,
                                    abc.ctypes.data_as(ctypes.c_void_p), len(sched), 1e-7, ws.data_ptr(), ws.numel(),
                                    _stream(dev)), lib)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("name", ["wide", "tall", "square", "zero"])
def test_newton_schulz_matches_reference_golden(dev, lib, name):
    z = np.load(os.path.join(GOLDEN, "muon_ns.npz"))
    sched = z["abc_" + name] if "abc_" + name in z else np.array(orc.NS_STANDARD)
    got = _ns_gpu(dev, lib, z["in_" + name], sched)[0]
    ref = z["out_" + name]
    assert np.linalg.norm(got - ref) <= NS_REL * max(np.linalg.norm(ref), 1e-30), name
    o = orc.newton_schulz(z["in_" + name], sched)
    assert np.linalg.norm(got - o) <= NS_REL * max(np.linalg.norm(o), 1e-30), name


@pytest.mark.parametrize("shape", [(3, 256, 384), (2, 320, 136), (1, 130, 70), (2, 512, 1280)])
def test_newton_schulz_batched_matches_oracle(dev, lib, shape):
    rng = np.random.default_rng(sum(shape))
    m = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    got = _ns_gpu(dev, lib, m, orc.NS_STANDARD)
    for i in range(shape[0]):
        o = orc.newton_schulz(m[i])
        rel = np.linalg.norm(got[i] - o) / np.linalg.norm(o)
        assert rel <= NS_REL, "batch item %d rel %.3e" % (i, rel)
        s = np.linalg.svd(got[i].astype(np.float64), compute_uv=False)
        assert s.max() < 1.3


def test_newton_schulz_large_batch_matches_oracle(dev, lib):
    """28 items of 1024 x 1024: the symmetric products (lower-triangle tiles,
    mirrored) and the third product all run on the 256 x 256 tile kernel."""
    rng = np.random.default_rng(1024)
    m = (rng.standard_normal((28, 1024, 1024)) * 1e-3).astype(np.float32)
    got = _ns_gpu(dev, lib, m, orc.NS_STANDARD)
    for i in (0, 13, 27):
        o = orc.newton_schulz(m[i])
        rel = np.linalg.norm(got[i] - o) / np.linalg.norm(o)
        assert rel <= NS_REL, "batch item %d rel %.3e" % (i, rel)
        s = np.linalg.svd(got[i].astype(np.float64), compute_uv=False)
        assert s.max() < 1.3


def test_newton_schulz_fp32_input(dev, lib):
    rng = np.random.default_rng(3)
    m = (rng.standard_normal((96, 160)) * 1e-2).astype(np.float32)
    got = _ns_gpu(dev, lib, m, orc.NS_STANDARD, torch.float32)[0]
    o = orc.newton_schulz(m)
    assert np.linalg.norm(got - o) <= NS_REL * np.linalg.norm(o)


@pytest.mark.parametrize("dtype", [orc.BF16, orc.F32])
@pytest.mark.parametrize("device_scalars", [False, True])
def test_normuon_and_apply_match_oracle(dev, lib, dtype, device_scalars):
    """device_scalars: the capturable form (step counter and the scalar row
    [lr, -, -, 1 - lr*wd] read on the device) gives the same result."""
    from gefen.kernels import automatic_gefen_fused as fused
    td = TORCH_DT[dtype]
    rng = np.random.default_rng(9)
    R, C = 72, 40
    upd = orc.bf16((rng.standard_normal((R, C)) * 0.1).astype(np.float32))
    p0 = orc.round_dtype((rng.standard_normal((R, C)) * 0.02).astype(np.float32), dtype)
    v0 = (rng.random(R) * 1e-4).astype(np.float32)
    ud = torch.from_numpy(upd).to(torch.bfloat16).to(dev)
    vd = torch.from_numpy(v0.copy()).to(dev)
    scale = torch.empty(R, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(int(lib.gefenx_normuon_workspace_bytes(R)), dtype=torch.uint8, device=dev)
    lr, wd = 1e-3, 0.01
    ratio = orc.adjust_lr_ratio("match_rms_adamw", (R, C))
    adj = lr * ratio
    step_dev = torch.full((), 3.0, dtype=torch.float32, device=dev) if device_scalars else None
    row = (torch.tensor([np.float32(lr), 1.0, 1.0, np.float32(1.0 - lr * wd)], dtype=torch.float32, device=dev)
           if device_scalars else None)
    _check(lib.gefenx_normuon_scale(ud.data_ptr(), R, C, vd.data_ptr(), 0.95, 0 if device_scalars else 3, 1e-8,
                                    scale.data_ptr(), ws.data_ptr(), ws.numel(),
                                    step_dev.data_ptr() if device_scalars else None, _stream(dev)), lib)
    pd = torch.from_numpy(p0.copy()).to(td).to(dev)
    _check(lib.gefenx_muon_apply(pd.data_ptr(), fused._dtype_code(td), ud.data_ptr(), scale.data_ptr(), R, C,
                                 0.0 if device_scalars else lr, wd, 0.0 if device_scalars else adj,
                                 row.data_ptr() if device_scalars else None, ratio, _stream(dev)), lib)
    torch.cuda.synchronize()
    o2, v = orc.normuon(upd, v0, 3)
    np.testing.assert_allclose(vd.cpu().numpy(), v, rtol=1e-6)
    p_ref = orc.muon_apply(p0, o2, dtype, lr, wd, adj)
    got = pd.float().cpu().numpy()
    # the float64-summed row norms may move one row's bf16 scale by an ulp
    assert np.mean(got == p_ref) > 0.97
    np.testing.assert_allclose(got, p_ref, rtol=0, atol=adj * 2.0 ** -7 + np.abs(p_ref).max() * 2.0 ** -7)


def _ulp(x, dtype):
    bits = 7 if dtype == orc.BF16 else 23
    e = np.floor(np.log2(np.maximum(np.abs(x), 2.0 ** -126)))
    return 2.0 ** (e - bits)


def _assert_update_close(got, ref, adj, dtype, msg):
    """Newton-Schulz on another GEMM order moves the update within the
    reference's rel-L2 2e-2 (||ortho||_F <= 1.3 sqrt(min(R, C))); p rounds."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    lim = adj * NS_REL * 1.3 * np.sqrt(min(got.shape)) + np.linalg.norm(_ulp(np.maximum(np.abs(got), np.abs(ref)), dtype))
    d = np.linalg.norm(got - ref)
    assert d <= lim, "%s: ||dp|| %.3e > %.3e" % (msg, d, lim)


MUON_KW = {
    "muon_bf16": (orc.BF16, dict(lr=0.02, weight_decay=0.1, momentum=0.95, nesterov=True), 4),
    "muon_f32": (orc.F32, dict(lr=0.02, weight_decay=0.1, momentum=0.9, nesterov=False,
                               adjust_lr_fn="match_rms_adamw", normuon=True), 3),
}


@pytest.mark.parametrize("case", list(MUON_KW))
def test_gefen_muon_class_matches_reference_golden(dev, case):
    """GefenMuon.step against the reference's GefenMuon(fused=False) step:
    indices and magnitudes bit-exact; parameters within the Newton-Schulz
    bound (each step starts from the reference's parameters)."""
    from gefen import GefenMuon
    dtype, kw, steps = MUON_KW[case]
    td = TORCH_DT[dtype]
    z = np.load(os.path.join(GOLDEN, case + ".npz"))
    names = ["a", "b"]
    ps = [(n, torch.nn.Parameter(torch.from_numpy(z["p0_" + n]).to(td).to(dev))) for n in names]
    opt = GefenMuon(ps, **kw)
    opt._gefen_codebook = torch.from_numpy(z["codebook"]).to(dev)
    for n, p in ps:
        opt.state[p]["automatic_period"] = int(z["period_" + n])
    for s in range(1, steps + 1):
        for n, p in ps:
            p.grad = torch.from_numpy(z["g%d_%s" % (s, n)]).to(td).to(dev)
        opt.step()
        torch.cuda.synchronize()
        for n, p in ps:
            st = opt.state[p]
            tag = "%s step %d %s" % (case, s, n)
            np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), z["idx%d_%s" % (s, n)],
                                          err_msg=tag + " indices")
            np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), z["mag%d_%s" % (s, n)],
                                          err_msg=tag + " magnitudes")
            adj = kw["lr"] * orc.adjust_lr_ratio(kw.get("adjust_lr_fn"), p.shape)
            ref = z["p%d_%s" % (s, n)]
            _assert_update_close(p.detach().float().cpu().numpy(), ref, adj, dtype, tag + " params")
            if "nv%d_%s" % (s, n) in z:
                nv = st["normuon_v"].cpu().numpy().reshape(-1)
                nv_ref = z["nv%d_%s" % (s, n)]
                assert np.linalg.norm(nv - nv_ref) <= 2 * NS_REL * np.linalg.norm(nv_ref), tag + " normuon_v"
                st["normuon_v"].copy_(torch.from_numpy(nv_ref).reshape(-1, 1).to(dev))
            p.data.copy_(torch.from_numpy(ref).to(td).to(dev))


def test_gefen_muon_hybrid_matches_reference_golden(dev):
    """GefenMuonHybrid with its defaults against the reference's hybrid step."""
    from gefen import GefenMuonHybrid
    z = np.load(os.path.join(GOLDEN, "hybrid_bf16.npz"))
    muon_names = ["layers.0.mlp.w", "layers.0.attn.o"]
    backup_names = ["embed_tokens.weight", "layers.0.norm.weight"]
    mk = lambda n: torch.nn.Parameter(torch.from_numpy(z["p0_" + n]).to(torch.bfloat16).to(dev))
    muon = [(n, mk(n)) for n in muon_names]
    backup = [(n, mk(n)) for n in backup_names]
    opt = GefenMuonHybrid(muon, backup, lr=1e-3, weight_decay=0.01)
    cb = torch.from_numpy(z["codebook"]).to(dev)
    opt.muon._gefen_codebook = cb.clone()
    opt.backup._gefen_codebook = cb.clone()
    named = dict(muon + backup)
    for n in muon_names + backup_names:
        opt.state[named[n]]["automatic_period"] = int(z["period_" + n])
    for s in range(1, 4):
        for n, p in named.items():
            p.grad = torch.from_numpy(z["g%d_%s" % (s, n)]).to(torch.bfloat16).to(dev)
        opt.step()
        torch.cuda.synchronize()
        for n, p in named.items():
            st = opt.state[p]
            tag = "hybrid step %d %s" % (s, n)
            np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), z["idx%d_%s" % (s, n)],
                                          err_msg=tag + " indices")
            np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), z["mag%d_%s" % (s, n)],
                                          err_msg=tag + " magnitudes")
            ref = z["p%d_%s" % (s, n)]
            got = p.detach().float().cpu().numpy()
            if n in muon_names:
                adj = 1e-3 * orc.adjust_lr_ratio("match_rms_adamw", p.shape)
                _assert_update_close(got, ref, adj, orc.BF16, tag + " params")
                st["normuon_v"].copy_(torch.from_numpy(z["normuon_v%d_%s" % (s, n)]).reshape(-1, 1).to(dev))
            else:
                np.testing.assert_allclose(st["vmean"].cpu().numpy().reshape(-1), z["vmean%d_%s" % (s, n)], rtol=1e-6)
                lim = _ulp(np.maximum(np.abs(got), np.abs(ref)), orc.BF16)
                assert (np.abs(got - ref) <= lim).all(), tag + " params"
            p.data.copy_(torch.from_numpy(ref).to(torch.bfloat16).to(dev))
    sd = opt.state_dict()
    assert set(sd) == {"muon", "backup", "backup_optimizer"} and sd["backup_optimizer"] == "gefen"


@pytest.mark.parametrize("case", [(orc.BF16, 96 * 40, 96, True), (orc.F32, 3000, 24, False)],
                         ids=lambda c: "dt%d-n%d-P%d-nest%d" % c)
def test_muon_momentum_stochastic_rounding_matches_oracle(dev, lib, case):
    """stochastic_round=1: indices, magnitudes and dense momentum bit-exact
    against oracle.muon_momentum(sr_seed=...) (SplitMix64 keyed by the flat
    element index, kernels/automatic_gefen_fused_kernel.cu:924)."""
    dtype, numel, period, nesterov = case
    from gefen.kernels import _native
    from gefen.kernels import automatic_gefen_fused as fused
    td = TORCH_DT[dtype]
    rng = np.random.default_rng(numel + 7)
    cb = np.load(os.path.join(GOLDEN, "learn.npz"))["cb"].astype(np.float32)
    qt = fused.quant_table(torch.from_numpy(cb).to(dev), td)
    idx_np, mag_np = _mom_state(numel, period, 2)
    idx = torch.from_numpy(idx_np.copy()).to(dev)
    mag = torch.from_numpy(mag_np.copy()).to(dev)
    ws = torch.zeros(int(lib.gefenx_workspace_bytes(_native.WS_MOMENTUM, 0, 0, numel // period)) + 256,
                     dtype=torch.uint8, device=dev)
    for step in range(3):
        seed = (1 << 33) + 17 * step
        g = torch.from_numpy((rng.standard_normal(numel) * 1e-3).astype(np.float32)).to(td)
        out = torch.empty(numel, dtype=td, device=dev)
        gd = g.to(dev)
        _check(lib.gefenx_quantized_momentum_update(gd.data_ptr(), fused._dtype_code(td), numel, period,
                                                    idx.data_ptr(), mag.data_ptr(), qt.data_ptr(), out.data_ptr(),
                                                    0.95, 1, seed, None, 1 if nesterov else 0, ws.data_ptr(),
                                                    ws.numel(), _stream(dev)), lib)
        torch.cuda.synchronize()
        idx_np, mag_np, out_np = orc.muon_momentum(g.float().numpy(), idx_np, mag_np, period, cb, dtype, 0.95,
                                                   nesterov, sr_seed=seed)
        tag = "sr step %d %s" % (step, case)
        np.testing.assert_array_equal(idx.cpu().numpy(), idx_np, err_msg=tag + " indices")
        np.testing.assert_array_equal(mag.cpu().numpy(), mag_np, err_msg=tag + " magnitudes")
        np.testing.assert_array_equal(out.float().cpu().numpy(), out_np, err_msg=tag + " momentum")


def _ns_torch_fp32(m, sched, eps=1e-7):
    """The oracle's Newton-Schulz statement (gefen_muon.py:236-291: every
    product and elementwise result rounded to bf16) with fp32 GEMMs on the
    device (torch fp32 matmul on contiguous operands) instead of float64 on
    the host -- for shapes the host cannot run in seconds."""
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


@pytest.mark.parametrize("shape", [(4096, 14336), (14336, 4096)])
def test_newton_schulz_workload_shape(dev, lib, shape):
    """Llama-3-8B down / gate projection shapes (the Gram product has K =
    14336, 224 K-steps of 64): within the reference's batched-vs-serial bound
    (rel. Frobenius 2e-2) of an fp32-GEMM restatement, and every singular
    value of the result in (0.5, 1.3)."""
    rng = np.random.default_rng(shape[0])
    m = torch.from_numpy((rng.standard_normal((2,) + shape) * 1e-3).astype(np.float32)).to(dev)
    from gefen.kernels import automatic_gefen_fused as fused
    b, r, c = m.shape
    x = m.to(torch.bfloat16)
    out = torch.empty(b, r, c, dtype=torch.bfloat16, device=dev)
    ws = torch.empty(int(lib.gefenx_ns_workspace_bytes(b, r, c)), dtype=torch.uint8, device=dev)
    abc = np.ascontiguousarray(np.asarray(orc.NS_STANDARD, np.float64).reshape(-1))
    _check(lib.gefenx_newton_schulz(x.data_ptr(), fused._dtype_code(torch.bfloat16), out.data_ptr(), b, r, c,
                                    abc.ctypes.data_as(ctypes.c_void_p), 5, 1e-7, ws.data_ptr(), ws.numel(),
                                    _stream(dev)), lib)
    torch.cuda.synchronize()
    for i in range(b):
        got = out[i].float()
        ref = _ns_torch_fp32(m[i], orc.NS_STANDARD)
        rel = (torch.linalg.vector_norm((got - ref).double()) / torch.linalg.vector_norm(ref.double())).item()
        assert rel <= NS_REL, "item %d rel %.3e" % (i, rel)
        small = got if got.shape[0] <= got.shape[1] else got.t().contiguous()
        gram = (small @ small.t().contiguous()).double().cpu().numpy()
        sv = np.sqrt(np.clip(np.linalg.eigvalsh(gram), 0.0, None))
        assert 0.5 < sv.min() and sv.max() < 1.3, (i, sv.min(), sv.max())


def test_newton_schulz_aspect_ratio_matches_oracle(dev, lib):
    """1024 x 3584 (the down projection's aspect ratio at oracle size)
    against the float64 oracle."""
    rng = np.random.default_rng(3584)
    m = (rng.standard_normal((1, 1024, 3584)) * 1e-3).astype(np.float32)
    got = _ns_gpu(dev, lib, m, orc.NS_STANDARD)[0]
    o = orc.newton_schulz(m[0])
    assert np.linalg.norm(got - o) <= NS_REL * np.linalg.norm(o)
    s = np.linalg.svd(got.astype(np.float64), compute_uv=False)
    assert 0.5 < s.min() and s.max() < 1.3


@pytest.mark.parametrize("case", list(MUON_KW))
def test_gefen_muon_strided_views_match_reference_golden(dev, case):
    """The reference's GefenMuon trajectory with every parameter and grad
    passed as a transposed view (storage [cols, rows], strides (1, rows)):
    the batched momentum reads the grads and the batched apply writes the
    parameters in place through their strides -- indices and magnitudes
    bit-exact, parameters within the Newton-Schulz bound."""
    from gefen import GefenMuon
    dtype, kw, steps = MUON_KW[case]
    td = TORCH_DT[dtype]
    z = np.load(os.path.join(GOLDEN, case + ".npz"))
    names = ["a", "b"]

    def view(a):  # the values of `a` in a transposed-view tensor
        return torch.from_numpy(np.ascontiguousarray(a.T)).to(td).to(dev).t()

    ps = [(n, torch.nn.Parameter(view(z["p0_" + n]))) for n in names]
    assert all(p.stride() == (1, p.shape[0]) for _, p in ps)
    opt = GefenMuon(ps, **kw)
    opt._gefen_codebook = torch.from_numpy(z["codebook"]).to(dev)
    for n, p in ps:
        opt.state[p]["automatic_period"] = int(z["period_" + n])
    for s in range(1, steps + 1):
        for n, p in ps:
            p.grad = view(z["g%d_%s" % (s, n)])
        opt.step()
        torch.cuda.synchronize()
        for n, p in ps:
            st = opt.state[p]
            tag = "%s strided step %d %s" % (case, s, n)
            np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), z["idx%d_%s" % (s, n)],
                                          err_msg=tag + " indices")
            np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), z["mag%d_%s" % (s, n)],
                                          err_msg=tag + " magnitudes")
            adj = kw["lr"] * orc.adjust_lr_ratio(kw.get("adjust_lr_fn"), p.shape)
            ref = z["p%d_%s" % (s, n)]
            _assert_update_close(p.detach().float().cpu().numpy(), ref, adj, dtype, tag + " params")
            if "nv%d_%s" % (s, n) in z:
                st["normuon_v"].copy_(torch.from_numpy(z["nv%d_%s" % (s, n)]).reshape(-1, 1).to(dev))
            p.data.copy_(view(ref))
            assert p.stride() == (1, p.shape[0])


def test_momentum_batch_over_several_launches_matches_oracle(dev, lib):
    """gefenx_muon_momentum_batch over 21 matrices of one shape (two launch
    sets of 16 and 5, mixed periods, one strided grad making a third, general
    run): every matrix's indices, magnitudes and momentum bit-exact against
    oracle.muon_momentum."""
    from gefen.kernels import _native
    from gefen.kernels import automatic_gefen_fused as fused
    rows, cols, n = 40, 96, 21
    numel = rows * cols
    rng = np.random.default_rng(7)
    cb = np.load(os.path.join(GOLDEN, "learn.npz"))["cb"].astype(np.float32)
    qt = fused.quant_table(torch.from_numpy(cb).to(dev), torch.bfloat16)
    periods = [768 if i % 3 else 3840 for i in range(n)]
    items = (_native.MuonItem * n)()
    keep = []
    state = []
    for i in range(n):
        idx_np, mag_np = _mom_state(numel, periods[i], i + 2)
        idx = torch.from_numpy(idx_np.copy()).to(dev)
        mag = torch.from_numpy(mag_np.copy()).to(dev)
        ws = torch.zeros(int(lib.gefenx_workspace_bytes(_native.WS_MOMENTUM, 0, 0, numel // periods[i])),
                         dtype=torch.uint8, device=dev)
        g_np = (rng.standard_normal((rows, cols)) * 1e-3).astype(np.float32)
        if i == 18:  # a transposed-view grad
            g = torch.from_numpy(np.ascontiguousarray(g_np.T)).to(torch.bfloat16).to(dev).t()
        else:
            g = torch.from_numpy(g_np).to(torch.bfloat16).to(dev)
        it = items[i]
        it.grad = g.data_ptr()
        it.grad_stride0, it.grad_stride1 = g.stride()
        it.m_codebook, it.m_magnitude, it.period = idx.data_ptr(), mag.data_ptr(), periods[i]
        it.workspace, it.workspace_bytes = ws.data_ptr(), ws.numel()
        keep += [g, idx, mag, ws]
        state.append((g, idx, mag, idx_np, mag_np))
    out = torch.empty(n, rows, cols, dtype=torch.bfloat16, device=dev)
    _check(lib.gefenx_muon_momentum_batch(items, n, fused._dtype_code(torch.bfloat16), rows, cols, qt.data_ptr(),
                                          out.data_ptr(), 0.95, 0, 0, None, 1, _stream(dev)), lib)
    torch.cuda.synchronize()
    for i, (g, idx, mag, idx_np, mag_np) in enumerate(state):
        ri, rm, ro = orc.muon_momentum(g.float().cpu().numpy(), idx_np, mag_np, periods[i], cb, orc.BF16, 0.95, True)
        tag = "matrix %d" % i
        np.testing.assert_array_equal(idx.cpu().numpy().reshape(-1), ri, err_msg=tag + " indices")
        np.testing.assert_array_equal(mag.cpu().numpy().reshape(-1), rm, err_msg=tag + " magnitudes")
        np.testing.assert_array_equal(out[i].float().cpu().numpy().reshape(-1), ro, err_msg=tag + " momentum")


def test_normuon_and_apply_batch_match_single_matrix_calls(dev, lib):
    """The batched NorMuon scale and apply over 18 matrices (two launch sets;
    one transposed-view parameter) give the single-matrix entry points'
    results bit for bit, and each matrix's normuon_v (1e-6) and parameters
    (bit for bit) equal oracle.normuon / oracle.muon_apply."""
    from gefen.kernels import _native
    rows, cols, n = 48, 64, 18
    rng = np.random.default_rng(3)
    upd = torch.from_numpy((rng.standard_normal((n, rows, cols)) * 0.05).astype(np.float32)).to(torch.bfloat16).to(dev)
    p0 = (rng.standard_normal((n, rows, cols)) * 0.02).astype(np.float32)
    v0 = (np.abs(rng.standard_normal((n, rows))) * 1e-3).astype(np.float32)
    items = (_native.MuonItem * n)()
    pb, vb = [], []
    for i in range(n):
        if i == 17:
            p = torch.from_numpy(np.ascontiguousarray(p0[i].T)).to(torch.bfloat16).to(dev).t()
        else:
            p = torch.from_numpy(p0[i]).to(torch.bfloat16).to(dev)
        v = torch.from_numpy(v0[i].copy()).to(dev)
        items[i].param = p.data_ptr()
        items[i].param_stride0, items[i].param_stride1 = p.stride()
        items[i].normuon_v = v.data_ptr()
        items[i].normuon_step = 3
        pb.append(p)
        vb.append(v)
    scale = torch.empty(n, rows, dtype=torch.bfloat16, device=dev)
    nws = torch.empty(int(lib.gefenx_normuon_batch_workspace_bytes(n, rows)), dtype=torch.uint8, device=dev)
    _check(lib.gefenx_normuon_scale_batch(items, n, upd.data_ptr(), rows, cols, 0.95, 1e-8, scale.data_ptr(),
                                          nws.data_ptr(), nws.numel(), _stream(dev)), lib)
    _check(lib.gefenx_muon_apply_batch(items, n, 2, upd.data_ptr(), scale.data_ptr(), rows, cols, 0.02, 0.1,
                                       0.02 * 0.2 * 8.0, 1.0, None, _stream(dev)), lib)
    for i in range(n):
        p = torch.from_numpy(p0[i]).to(torch.bfloat16).to(dev)
        v = torch.from_numpy(v0[i].copy()).to(dev)
        sc = torch.empty(rows, dtype=torch.bfloat16, device=dev)
        ws = torch.empty(int(lib.gefenx_normuon_workspace_bytes(rows)), dtype=torch.uint8, device=dev)
        _check(lib.gefenx_normuon_scale(upd[i].data_ptr(), rows, cols, v.data_ptr(), 0.95, 3, 1e-8, sc.data_ptr(),
                                        ws.data_ptr(), ws.numel(), None, _stream(dev)), lib)
        _check(lib.gefenx_muon_apply(p.data_ptr(), 2, upd[i].data_ptr(), sc.data_ptr(), rows, cols, 0.02, 0.1,
                                     0.02 * 0.2 * 8.0, None, 1.0, _stream(dev)), lib)
        torch.cuda.synchronize()
        assert torch.equal(sc, scale[i]), i
        assert torch.equal(v, vb[i]), i
        assert torch.equal(p, pb[i].contiguous()), i
        # and the batched result against the oracle directly
        u_ref, v_ref = orc.normuon(upd[i].float().cpu().numpy(), v0[i], 3, 0.95, 1e-8)
        p_start = torch.from_numpy(p0[i]).to(torch.bfloat16).float().numpy()
        p_ref = orc.muon_apply(p_start, u_ref, orc.BF16, 0.02, 0.1, 0.02 * 0.2 * 8.0)
        np.testing.assert_allclose(vb[i].cpu().numpy(), v_ref, rtol=1e-6, err_msg="matrix %d normuon_v" % i)
        np.testing.assert_array_equal(pb[i].float().cpu().numpy(), p_ref, err_msg="matrix %d params" % i)


@pytest.mark.parametrize("shape", [(96, 256), (256, 96), (64, 200)])
def test_newton_schulz_normalisation_is_exact(dev, lib, shape):
    """An empty schedule returns the normalised X = bf16(bf16(G) / bf16(||G||))
    itself: bit-exact against the oracle's float32 division (the kernel divides
    through the reciprocal with a correction step; zeros, tiny values and a
    denominator of awkward mantissa must all round as the true quotient)."""
    gen = np.random.default_rng(11)
    m = gen.standard_normal(shape).astype(np.float32) * np.float32(3.0)
    m[0, :5] = 0.0
    m[1, :3] = -0.0
    m[2, :4] = np.float32(1e-32)
    m[3, :7] = gen.standard_normal(7).astype(np.float32) * np.float32(1e-29)
    print("ns normalisation", shape, flush=True)
    out = _ns_gpu(dev, lib, m[None], [])[0]
    ref = orc.newton_schulz(m, [])
    np.testing.assert_array_equal(out.view(np.uint32), ref.astype(np.float32).view(np.uint32))
