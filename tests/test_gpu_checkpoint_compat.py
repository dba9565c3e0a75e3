"""Resume on MI355X from checkpoints the reference wrote, and from our own.

tests/golden/ckpt_<case>.pt is the reference's Gefen.state_dict() after three
CPU steps (period search and codebook learned by the reference); the .npz
holds the trajectory the reference itself takes after loading it into a
fresh optimizer and stepping three more grads (gefen.py:5456-5707).  Loaded
here into this build's Gefen on the GPU, the continued trajectory must match
the reference's: indices and magnitudes bit-exact, second moments within
1e-6, parameters within one bf16 ulp.

Round trip: a bf16 run interrupted by state_dict / load_state_dict into a
fresh optimizer continues exactly like the uninterrupted run (the fp32 state
must not pass through the parameters' bf16 on load).
"""
import copy
import os

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import assert_within_ulp

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


@pytest.mark.parametrize("case", ["fact_bf16", "block_bf16"])
@pytest.mark.parametrize("capturable", [False, True])
def test_resume_from_reference_checkpoint(dev, case, capturable):
    from gefen import Gefen
    print("resume reference checkpoint", case, "capturable", capturable, flush=True)
    sd = torch.load(os.path.join(GOLD, "ckpt_%s.pt" % case), weights_only=True)
    ref = np.load(os.path.join(GOLD, "ckpt_%s.npz" % case))
    pre, steps = int(ref["pre"]), int(ref["steps"])
    names = ("w", "b")
    params = [(n, torch.nn.Parameter(torch.from_numpy(ref["p%d_%s" % (pre, n)]).to(torch.bfloat16).to(dev)))
              for n in names]
    opt = Gefen(params, lr=6e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=float(ref["wd"]),
                factored_v_2d=bool(ref["factored"]), capturable=capturable)
    opt.load_state_dict(copy.deepcopy(sd))
    for s in range(pre + 1, steps + 1):
        for n, p in params:
            p.grad = torch.from_numpy(ref["g%d_%s" % (s, n)]).to(torch.bfloat16).to(dev)
        opt.step()
        torch.cuda.synchronize()
        for n, p in params:
            st = opt.state[p]
            tag = "%s step %d %s" % (case, s, n)
            np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), ref["idx%d_%s" % (s, n)],
                                          err_msg=tag)
            np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), ref["mag%d_%s" % (s, n)],
                                          err_msg=tag)
            for key in ("v_row", "v_col", "vmean"):
                k = "%s%d_%s" % (key, s, n)
                if k in ref:
                    np.testing.assert_allclose(st[key].cpu().numpy().reshape(-1), ref[k], rtol=1e-6, err_msg=tag)
            assert_within_ulp(p.detach().float().cpu().numpy(), ref["p%d_%s" % (s, n)], orc.BF16, tag,
                              atol=1e-6 * 6e-5)
    assert opt.state_dict()["gefen_global_step"] == int(ref["global_step"])


@pytest.mark.parametrize("factored", [True, False])
def test_bf16_round_trip_continues_exactly(dev, factored):
    from gefen import Gefen
    print("round trip factored", factored, flush=True)
    gen = torch.Generator().manual_seed(3)
    shapes = [("w", (96, 160)), ("b", (160,))]
    init = [(n, torch.randn(*s, generator=gen) * 0.02) for n, s in shapes]
    grads = [[torch.randn(*s, generator=gen) * 1e-3 for _, s in shapes] for _ in range(6)]

    def make(values):
        ps = [(n, torch.nn.Parameter(v.to(torch.bfloat16).to(dev))) for n, v in values]
        return ps, Gefen(ps, lr=1e-3, weight_decay=0.01, factored_v_2d=factored)

    def run(ps, opt, steps):
        for gs in steps:
            for (_, p), g in zip(ps, gs):
                p.grad = g.to(torch.bfloat16).to(dev)
            opt.step()

    ps_a, a = make(init)
    run(ps_a, a, grads)
    ps_b, b = make(init)
    run(ps_b, b, grads[:3])
    sd = copy.deepcopy(b.state_dict())
    ps_c, c = make([(n, p.detach().float().cpu()) for n, p in ps_b])
    c.load_state_dict(sd)
    run(ps_c, c, grads[3:])
    torch.cuda.synchronize()
    for (n, pa), (_, pc) in zip(ps_a, ps_c):
        sa, sc = a.state[pa], c.state[pc]
        for k in ("m_codebook", "m_magnitude", "v_row", "v_col", "vmean"):
            if k in sa:
                assert sc[k].dtype == sa[k].dtype, (n, k)
                if k in ("m_codebook", "m_magnitude"):
                    assert torch.equal(sa[k], sc[k]), (n, k)
                else:
                    torch.testing.assert_close(sc[k], sa[k], rtol=1e-6, atol=0)
        torch.testing.assert_close(pc.detach().float(), pa.detach().float(), rtol=2.0 ** -7, atol=1e-9)


def test_reset_to_a_fresh_state_follows_a_fresh_trajectory(dev):
    """Step, load the state_dict of a never-stepped optimizer (no codebook),
    step again: the run must equal a fresh optimizer's first steps exactly
    (the codebook and periods are learned again from the new step-1 grads)."""
    from gefen import Gefen
    gen = torch.Generator().manual_seed(3)
    w0 = (torch.randn(64, 96, generator=gen) * 0.02).to(torch.bfloat16)
    b0 = (torch.randn(96, generator=gen) * 0.02).to(torch.bfloat16)
    grads = [((torch.randn(64, 96, generator=gen) * 1e-3).to(torch.bfloat16),
              (torch.randn(96, generator=gen) * 1e-2).to(torch.bfloat16)) for _ in range(5)]

    def make():
        ps = [("w", torch.nn.Parameter(w0.clone().to(dev))), ("b", torch.nn.Parameter(b0.clone().to(dev)))]
        return ps, Gefen(ps, lr=6e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)

    pa, oa = make()
    fresh_sd = oa.state_dict()
    for gw, gb in grads[:2]:  # an unrelated trajectory: learns a codebook from other grads
        pa[0][1].grad, pa[1][1].grad = gb.new_ones(64, 96).to(dev) * 1e-2, gb.to(dev) * 3
        oa.step()
    oa.load_state_dict(copy.deepcopy(fresh_sd))
    with torch.no_grad():
        pa[0][1].copy_(w0.to(dev))
        pa[1][1].copy_(b0.to(dev))
    pb, ob = make()
    for s, (gw, gb) in enumerate(grads[2:], start=1):
        for ps in (pa, pb):
            ps[0][1].grad, ps[1][1].grad = gw.to(dev), gb.to(dev)
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        assert torch.equal(oa._gefen_codebook, ob._gefen_codebook), s
        for (_, x), (_, y) in zip(pa, pb):
            sa, sb = oa.state[x], ob.state[y]
            assert sa["automatic_period"] == sb["automatic_period"]
            assert torch.equal(sa["m_codebook"], sb["m_codebook"]), s
            assert torch.equal(sa["m_magnitude"], sb["m_magnitude"]), s
            assert torch.equal(x, y), s
