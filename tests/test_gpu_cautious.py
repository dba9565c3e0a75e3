"""Cautious masking of the Muon update on MI355X (gefen_muon.py:396-405,
1148-1162): the agreement counts and the masked apply through the C ABI,
bit-exact against oracle.muon_apply(p, oracle.cautious_mask(u', grad)) with
u' the NorMuon-scaled update; contiguous and transposed grads, rows of 8k
and of other widths (the chunked and the element kernels), three parameter
dtypes; then GefenMuon(cautious=True) along the reference's golden grads
against the oracle's trajectory within the Newton-Schulz bound."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TORCH_DT = {orc.F32: torch.float32, orc.F16: torch.float16, orc.BF16: torch.bfloat16}
NS_REL = 2e-2


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


@pytest.fixture(scope="module")
def lib():
    from gefen.kernels import _native
    return _native.load()


def _check(rc):
    from gefen.kernels import _native
    _native.check(rc, "call")


@pytest.mark.parametrize("dtype", [orc.BF16, orc.F32, orc.F16])
@pytest.mark.parametrize("shape", [(64, 96), (40, 36)])
@pytest.mark.parametrize("with_scale", [False, True])
def test_cautious_apply_matches_oracle(dev, lib, dtype, shape, with_scale):
    from gefen.kernels import _native
    rows, cols = shape
    n = 3
    td = TORCH_DT[dtype]
    rng = np.random.default_rng(7 + rows)
    upd = orc.bf16(rng.standard_normal((n, rows, cols)).astype(np.float32) * np.float32(0.1))
    g = orc.round_dtype(rng.standard_normal((n, rows, cols)).astype(np.float32) * np.float32(1e-3), dtype)
    g[0, 0, :9] = 0.0                                    # zero grads agree with nothing
    g[1, 1, :4] = np.float32(2.0 ** -70) * np.sign(upd[1, 1, :4])  # tiny: the promoted dtype decides
    upd[1, 1, :4] = np.float32(2.0 ** -70) * np.sign(upd[1, 1, :4] + 1e-30)
    g = orc.round_dtype(g, dtype)  # (fp16 flushes the tiny ones to zero)
    p0 = orc.round_dtype(rng.standard_normal((n, rows, cols)).astype(np.float32) * np.float32(0.02), dtype)
    scale = orc.bf16(rng.uniform(0.5, 2.0, (n, rows)).astype(np.float32)) if with_scale else None
    print("cautious", dtype, shape, with_scale, flush=True)
    ud = torch.from_numpy(upd).to(torch.bfloat16).to(dev)
    sd = torch.from_numpy(scale).to(torch.bfloat16).to(dev) if with_scale else None
    items = (_native.MuonItem * n)()
    ps, gs = [], []
    for i in range(n):
        if i == 2:  # a transposed-view grad
            gt = torch.from_numpy(np.ascontiguousarray(g[i].T)).to(td).to(dev).t()
        else:
            gt = torch.from_numpy(g[i]).to(td).to(dev)
        pt = torch.from_numpy(p0[i]).to(td).to(dev)
        items[i].grad = gt.data_ptr()
        items[i].grad_stride0, items[i].grad_stride1 = gt.stride()
        items[i].param = pt.data_ptr()
        items[i].param_stride0, items[i].param_stride1 = pt.stride()
        ps.append(pt)
        gs.append(gt)
    counts = torch.full((n,), -1, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    code = {orc.F32: 0, orc.F16: 1, orc.BF16: 2}[dtype]
    _check(lib.gefenx_muon_cautious_count_batch(items, n, code, ud.data_ptr(), sd.data_ptr() if with_scale else None,
                                                rows, cols, counts.data_ptr(), stream))
    lr, wd, adj = 0.02, 0.1, 0.02 * 0.2 * 8.0
    _check(lib.gefenx_muon_apply_batch(items, n, code, ud.data_ptr(), sd.data_ptr() if with_scale else None, rows,
                                       cols, lr, wd, adj, 1.0, counts.data_ptr(), stream))
    torch.cuda.synchronize()
    for i in range(n):
        u = upd[i] if scale is None else orc.bf16(upd[i] * scale[i][:, None])
        masked = orc.cautious_mask(u, g[i], dtype)
        prod = (u * g[i]).astype(np.float32)
        if dtype == orc.BF16:
            prod = orc.bf16(prod)
        assert int(counts[i]) == int((prod > 0).sum()), i
        ref = orc.muon_apply(p0[i], masked, dtype, lr, wd, adj)
        got = ps[i].float().cpu().numpy()
        np.testing.assert_array_equal(got.view(np.uint32), ref.astype(np.float32).view(np.uint32), err_msg=str(i))


def test_gefen_muon_cautious_follows_the_oracle_trajectory(dev):
    from gefen import GefenMuon
    z = np.load(os.path.join(GOLDEN, "muon_bf16.npz"))
    names = ["a", "b"]
    kw = dict(lr=0.02, weight_decay=0.1, momentum=0.95, nesterov=True)
    ps = [(n, torch.nn.Parameter(torch.from_numpy(z["p0_" + n]).to(torch.bfloat16).to(dev))) for n in names]
    opt = GefenMuon(ps, cautious=True, **kw)
    assert opt.param_groups[0]["cautious"] is True
    opt._gefen_codebook = torch.from_numpy(z["codebook"]).to(dev)
    cb = z["codebook"]
    st = {}
    for n, p in ps:
        per = int(z["period_" + n])
        opt.state[p]["automatic_period"] = per
        st[n] = dict(idx=np.zeros(p.numel(), np.uint8), mag=np.zeros(p.numel() // per, np.float32), per=per)
    for s in range(1, 5):
        for n, p in ps:
            p.grad = torch.from_numpy(z["g%d_%s" % (s, n)]).to(torch.bfloat16).to(dev)
        before = {n: p.detach().float().cpu().numpy() for n, p in ps}
        opt.step()
        torch.cuda.synchronize()
        for n, p in ps:
            g = z["g%d_%s" % (s, n)]
            o = st[n]
            o["idx"], o["mag"], mom = orc.muon_momentum(g, o["idx"], o["mag"], o["per"], cb, orc.BF16, 0.95, True)
            np.testing.assert_array_equal(opt.state[p]["m_codebook"].cpu().numpy().reshape(-1), o["idx"])
            ortho = orc.cautious_mask(orc.newton_schulz(mom.reshape(g.shape)), g, orc.BF16)
            adj = kw["lr"] * orc.adjust_lr_ratio(None, g.shape)
            ref = orc.muon_apply(before[n], ortho, orc.BF16, kw["lr"], kw["weight_decay"], adj)
            got = p.detach().float().cpu().numpy()
            # the step against the oracle's: within the Newton-Schulz bound of the update
            d_ref = ref - orc.muon_apply(before[n], np.zeros_like(ortho), orc.BF16, kw["lr"], kw["weight_decay"], 0.0)
            assert np.linalg.norm(got - ref) <= NS_REL * np.linalg.norm(d_ref) + 1e-6, (s, n)
            assert np.isfinite(got).all()


@pytest.mark.parametrize("dtype", [orc.F16, orc.BF16, orc.F32])
def test_standalone_cautious_mask_keeps_bf16_range(dev, dtype):
    """The standalone _cautious_mask_ (gefen_muon.py:396-405) on an update
    where only a handful of elements agree with the grad, so the kept ones
    are scaled by ~numel/8 (here 1024 x 4096 / 8 = 524288), and whose values
    reach 100: u * scale reaches ~5e7, beyond fp16's range but inside bf16's.
    Bit-exact against oracle.cautious_mask, finite, for every grad dtype."""
    from gefen.gefen_muon import _cautious_mask_
    gen = torch.Generator().manual_seed(3)
    rows, cols = 1024, 4096
    u = (torch.randn(rows, cols, generator=gen) * 30.0).clamp(-100, 100).to(torch.bfloat16)
    g = -u.float() * 1e-3  # every product negative ...
    flat = g.view(-1)
    agree = torch.randperm(rows * cols, generator=gen)[:8]
    flat[agree] = -flat[agree]  # ... except 8
    g = g.to(TORCH_DT[dtype])
    want = orc.cautious_mask(u.float().numpy(), g.float().numpy(), dtype)
    got = _cautious_mask_(u.clone().to(dev), g.to(dev))
    torch.cuda.synchronize()
    got_np = got.float().cpu().numpy()
    assert np.isfinite(got_np).all()
    assert float(np.abs(got_np).max()) > 65504.0  # past fp16's largest finite value
    np.testing.assert_array_equal(got_np, want)
