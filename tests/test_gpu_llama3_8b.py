"""BASELINE configs[1] on the GPU at full size: the Llama-3-8B-shaped bf16 set
(290 tensors, 8,030,257,152 params) that bench.py times, built and seeded the
same way (bench.make_params / bench.fill_grads), plain Gefen with
factored_v_2d, lr 6e-5, betas (0.9, 0.999), eps 1e-8, wd 0.01.

Five seeded warm-up steps (the first runs the GPU period search and learns
the codebook), then one more step is checked.  The oracle cannot step 8e9
elements in seconds, so the checks are local (tests/local_checks.py): for one
tensor of every class -- embedding, lm_head, q, k, v, o, gate, up, down -- the
first, middle and last momentum block at the tensor's searched period
(indices and magnitude bit-exact against oracle.momentum_update), sampled
rows' v_row, columns' v_col (1e-6 relative) and the rows' new parameters
(1 bf16 ulp); one RMSNorm vector whole through oracle.block_step (indices and
magnitudes bit-exact).  The periods of one k projection and one norm vector
are checked against oracle.find_period on their step-1 grads.
"""
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import FactoredProbe, assert_within_ulp

pytestmark = pytest.mark.gpu

LR, BETAS, EPS, WD = 6e-5, (0.9, 0.999), 1e-8, 0.01
WARMUP = 5

PROBED = {
    "model.embed_tokens.weight": "embed",
    "lm_head.weight": "lm_head",
    "model.layers.0.self_attn.q_proj.weight": "q",
    "model.layers.17.self_attn.k_proj.weight": "k",
    "model.layers.3.self_attn.v_proj.weight": "v",
    "model.layers.30.self_attn.o_proj.weight": "o",
    "model.layers.31.mlp.gate_proj.weight": "gate",
    "model.layers.12.mlp.up_proj.weight": "up",
    "model.layers.5.mlp.down_proj.weight": "down",
}
NORM = "model.layers.9.input_layernorm.weight"
PERIOD_CHECKED = ("model.layers.0.self_attn.k_proj.weight", "model.layers.2.post_attention_layernorm.weight")


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
    if free < 60 * (1 << 30):
        pytest.skip("needs about 60 GiB of free device memory")
    return torch.device("cuda", 0)


def test_llama3_8b_set_local_parity(dev):
    import bench
    from gefen import Gefen
    shapes = bench.llama3_8b_shapes()
    params = bench.make_params(torch, shapes, dev)
    byname = dict(params)
    opt = Gefen(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, factored_v_2d=True)
    step1_grads = {}
    for w in range(WARMUP):
        bench.fill_grads(torch, params, w, dev)
        if w == 0:
            step1_grads = {n: _f(byname[n].grad) for n in PERIOD_CHECKED}
        opt.step()
    torch.cuda.synchronize()
    _say("llama3-8b: %d warm-up steps done" % WARMUP)
    for n, g in step1_grads.items():
        assert opt.state[byname[n]]["automatic_period"] == orc.find_period(g, g.shape), n
    cb = opt._gefen_codebook.cpu().numpy()

    bench.fill_grads(torch, params, WARMUP, dev)
    probes = []
    for n, cls in PROBED.items():
        p = byname[n]
        st = opt.state[p]
        P = st["automatic_period"]
        R, C = p.shape
        nb = p.numel() // P
        rows = [0, 1, R // 2, (nb // 2) * P // C, R - 1]
        probe = FactoredProbe("%s (%s, P=%d)" % (cls, n, P), p, P, rows, [0, 7, C // 2, C - 1],
                              [0, nb // 2, nb - 1])
        probe.capture(st)
        probes.append(probe)
    pn = byname[NORM]
    sn = opt.state[pn]
    norm_in = (_f(pn), _f(pn.grad), sn["m_codebook"].cpu().numpy().reshape(-1),
               sn["m_magnitude"].cpu().numpy().reshape(-1), sn["vmean"].cpu().numpy().reshape(-1))
    opt.step()
    torch.cuda.synchronize()
    step = WARMUP + 1
    _say("llama3-8b: checked step %d done" % step)
    for probe in probes:
        probe.verify(opt.state[probe.p], cb, step=step, beta1=BETAS[0], beta2=BETAS[1], lr=LR, eps=EPS, wd=WD)
        _say("  %s ok" % probe.name)
    p0, g0, i0, m0, v0 = norm_in
    P = sn["automatic_period"]
    bc1, bc2 = 1 - BETAS[0] ** step, 1 - BETAS[1] ** step
    p1, i1, m1, v1 = orc.block_step(p0, g0, i0, m0, v0, P, cb, orc.BF16, beta1=BETAS[0], beta2=BETAS[1],
                                    lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=WD)
    np.testing.assert_array_equal(sn["m_codebook"].cpu().numpy().reshape(-1), i1, err_msg="norm indices")
    np.testing.assert_array_equal(sn["m_magnitude"].cpu().numpy().reshape(-1), m1, err_msg="norm magnitudes")
    np.testing.assert_allclose(sn["vmean"].cpu().numpy().reshape(-1), v1, rtol=1e-6, err_msg="norm vmean")
    assert_within_ulp(_f(pn), p1, orc.BF16, "norm p", atol=1e-6 * LR)
    _say("  norm (%s, P=%d) ok" % (NORM, P))
