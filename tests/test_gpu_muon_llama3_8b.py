"""BASELINE configs[3] on the GPU at full size: GefenMuonHybrid on the
Llama-3-8B layer stack that `bench.py --workload muon` times -- 224 hidden
matrices (4096 x 4096, 1024 x 4096, 14336 x 4096, 4096 x 14336) through the
quantised momentum and 5-step standard Newton-Schulz on bf16 MFMA, batched
16 per launch set; 66 norms, the embedding and lm_head through the
block-vmean Gefen backup.  bf16 params N(0, 0.02), grads N(0, 1e-3) from a
seed, lr 1e-3, wd 0.01, NorMuon and match_rms_adamw (the hybrid defaults).

Two warm-up steps, then one checked step whose stages are checked one by one
on the first matrix of every shape (layer 0's q, k, gate and down), each
from the GPU's own input to that stage, so a mismatch names its stage:
  - momentum: indices, magnitudes and the dense (Nesterov) momentum handed
    to Newton-Schulz bit-exact against oracle.muon_momentum (the dense
    momentum is recorded at the Newton-Schulz call inside the step);
  - Newton-Schulz: the GPU's output within the reference's 2e-2 relative
    Frobenius bound of the fp32 restatement, singular values below 1.3 (and
    above 0.5 for the rectangular shapes);
  - NorMuon: normuon_v within 1e-6 of oracle.normuon on the GPU's
    Newton-Schulz output;
  - apply: parameters within 1 bf16 ulp of oracle.muon_apply.
Backup: three embedding blocks through oracle.block_step and a whole
RMSNorm vector (indices and magnitudes bit-exact, vmean 1e-6, p 1 ulp).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import BlockProbe, assert_within_ulp, ns_torch_fp32

pytestmark = pytest.mark.gpu

LR, WD, BETA, NS_REL = 1e-3, 0.01, 0.95, 2e-2
WARMUP = 2
PROBED = ("model.layers.0.self_attn.q_proj.weight", "model.layers.0.self_attn.k_proj.weight",
          "model.layers.0.mlp.gate_proj.weight", "model.layers.0.mlp.down_proj.weight")
NORM = "model.layers.7.input_layernorm.weight"
EMBED = "model.embed_tokens.weight"


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _f(t):
    return t.detach().float().cpu().numpy()


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    free, _ = torch.cuda.mem_get_info(0)
    if free < 90 * (1 << 30):
        pytest.skip("needs about 90 GiB of free device memory")
    return torch.device("cuda", 0)


def _fill(params, seed, dev):
    gen = torch.Generator(device=dev).manual_seed(30_000 + seed)
    for _, p in params:
        if p.grad is None:
            p.grad = torch.empty_like(p)
        p.grad.normal_(0.0, 1e-3, generator=gen)


def test_muon_hybrid_llama3_8b_stages(dev, monkeypatch):
    import bench
    from gefen import GefenMuonHybrid
    from gefen import gefen_muon
    from gefen.params import is_muon_param
    params = bench.make_params(torch, bench.llama3_8b_shapes(), dev)
    byname = dict(params)
    muon = [(n, p) for n, p in params if is_muon_param(n, p)]
    backup = [(n, p) for n, p in params if not is_muon_param(n, p)]
    assert len(muon) == 224 and len(backup) == 66
    opt = GefenMuonHybrid(muon, backup, lr=LR, weight_decay=WD, ns_schedule="standard", ns_steps=5)
    for w in range(WARMUP):
        _fill(params, w, dev)
        opt.step()
    torch.cuda.synchronize()
    _say("muon llama3-8b: %d warm-up steps done" % WARMUP)

    _fill(params, WARMUP, dev)
    # the first matrix of each shape is item 0 of its shape's first launch set
    shapes = {tuple(byname[n].shape): n for n in PROBED}
    assert [n for n, _ in muon if tuple(byname[n].shape) == tuple(byname[PROBED[0]].shape)][0] == PROBED[0]
    before = {}
    for n in PROBED:
        p = byname[n]
        st = opt.muon.state[p]
        before[n] = dict(p=_f(p), g=_f(p.grad), idx=st["m_codebook"].cpu().numpy().reshape(-1),
                         mag=st["m_magnitude"].cpu().numpy().reshape(-1),
                         v=st["normuon_v"].cpu().numpy().reshape(-1), nstep=int(st["normuon_step"]),
                         P=int(st["automatic_period"]))
    recorded = {}
    original = gefen_muon._zeropower_via_newtonschulz_batched

    def recording(mom, *args, **kw):
        out = original(mom, *args, **kw)
        key = tuple(mom.shape[1:])
        if key in shapes and key not in recorded:
            recorded[key] = (mom[0].detach().clone(), out[0].detach().clone())
        return out

    monkeypatch.setattr(gefen_muon, "_zeropower_via_newtonschulz_batched", recording)
    bstate = opt.backup.state
    pe = byname[EMBED]
    eprobe = BlockProbe("embed (P=%d)" % bstate[pe]["automatic_period"], pe, bstate[pe]["automatic_period"],
                        [0, pe.numel() // bstate[pe]["automatic_period"] // 2, -1])
    eprobe.capture(bstate[pe])
    pn = byname[NORM]
    norm_in = (_f(pn), _f(pn.grad), bstate[pn]["m_codebook"].cpu().numpy().reshape(-1),
               bstate[pn]["m_magnitude"].cpu().numpy().reshape(-1), bstate[pn]["vmean"].cpu().numpy().reshape(-1))
    opt.step()
    torch.cuda.synchronize()
    monkeypatch.setattr(gefen_muon, "_zeropower_via_newtonschulz_batched", original)
    step = WARMUP + 1
    _say("muon llama3-8b: checked step %d done" % step)
    assert set(recorded) == set(shapes)

    cb = opt.muon._gefen_codebook.cpu().numpy()
    for n in PROBED:
        p = byname[n]
        b = before[n]
        st = opt.muon.state[p]
        shape = tuple(p.shape)
        mom_gpu, ortho_gpu = recorded[shape]
        # momentum: state and the dense momentum, bit for bit
        i1, m1, out = orc.muon_momentum(b["g"], b["idx"], b["mag"], b["P"], cb, orc.BF16, BETA, nesterov=True)
        np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), i1, err_msg=n + " indices")
        np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), m1, err_msg=n + " magnitudes")
        np.testing.assert_array_equal(mom_gpu.float().cpu().numpy().reshape(-1), out, err_msg=n + " momentum")
        # Newton-Schulz: the reference's bound against the fp32 restatement
        ref = ns_torch_fp32(mom_gpu.float(), orc.NS_STANDARD)
        got = ortho_gpu.float()
        rel = (torch.linalg.vector_norm((got - ref).double()) / torch.linalg.vector_norm(ref.double())).item()
        assert rel <= NS_REL, "%s Newton-Schulz rel %.3e" % (n, rel)
        small = got if got.shape[0] <= got.shape[1] else got.t().contiguous()
        sv = torch.linalg.eigvalsh((small.double() @ small.double().t())).clamp_min(0).sqrt()
        # every singular value below 1.3; above 0.5 too for the rectangular
        # shapes -- a square momentum's smallest singular values start near 0
        # and five steps lift them by at most 3.4445^5
        assert sv.max().item() < 1.3, (n, sv.max().item())
        if max(shape) >= 2 * min(shape):
            assert sv.min().item() > 0.5, (n, sv.min().item())
        # NorMuon and apply, from the GPU's Newton-Schulz output
        o_np = got.cpu().numpy()
        upd, v1 = orc.normuon(o_np, b["v"], b["nstep"] + 1, 0.95, 1e-8)
        np.testing.assert_allclose(st["normuon_v"].cpu().numpy().reshape(-1), v1, rtol=1e-6,
                                   err_msg=n + " normuon_v")
        adjusted = LR * orc.adjust_lr_ratio("match_rms_adamw", shape)
        p1 = orc.muon_apply(b["p"], upd, orc.BF16, LR, WD, adjusted)
        assert_within_ulp(_f(p), p1, orc.BF16, n + " p")
        _say("  %s %s ok (Newton-Schulz rel %.2e, sv %.3f..%.3f)" % (n, shape, rel, sv.min().item(),
                                                                     sv.max().item()))

    bcb = opt.backup._gefen_codebook.cpu().numpy()
    eprobe.verify(bstate[pe], bcb, step=step, beta1=0.9, beta2=0.999, lr=LR, eps=1e-8, wd=WD)
    _say("  %s ok" % eprobe.name)
    p0, g0, i0, m0, v0 = norm_in
    P = bstate[pn]["automatic_period"]
    bc1, bc2 = 1 - 0.9 ** step, 1 - 0.999 ** step
    p1, i1, m1, v1 = orc.block_step(p0, g0, i0, m0, v0, P, bcb, orc.BF16, beta1=0.9, beta2=0.999, lr=LR,
                                    eps=1e-8, bc1=bc1, bc2=bc2, wd=WD)
    np.testing.assert_array_equal(bstate[pn]["m_codebook"].cpu().numpy().reshape(-1), i1, err_msg="norm indices")
    np.testing.assert_array_equal(bstate[pn]["m_magnitude"].cpu().numpy().reshape(-1), m1, err_msg="norm mags")
    np.testing.assert_allclose(bstate[pn]["vmean"].cpu().numpy().reshape(-1), v1, rtol=1e-6, err_msg="norm vmean")
    assert_within_ulp(_f(pn), p1, orc.BF16, "norm p", atol=1e-6 * LR)
    _say("  %s (P=%d) ok" % (NORM, P))
