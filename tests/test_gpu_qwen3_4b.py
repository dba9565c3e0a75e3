"""BASELINE configs[2] on the GPU at full size: the Qwen3-4B-shaped bf16 set
that `bench.py --workload qwen` times (398 tensors, 4,022,468,096 params;
every 10th 2D tensor a transposed view of [C, R] storage, so each class
appears as a view), grads 1e-3 * StudentT(nu=3) from a seed, plain Gefen
with lr 6e-5, betas (0.9, 0.999), eps 1e-8, wd 0.01, factored_v_2d on and
off.

Two seeded warm-up steps (the first runs the GPU period search and learns
the codebook), then one checked step.  The oracle cannot step 4e9 elements
in seconds, so the checks are local (tests/local_checks.py), one tensor per
class at its searched period: the tied 151936 x 2560 embedding, contiguous
q / o / up projections, and transposed k (1024 x 2560), gate (9728 x 2560),
o (2560 x 4096) and down (2560 x 9728) views.  Factored on: the first,
middle and last momentum block (indices and magnitude bit-exact), sampled
rows' v_row and columns' v_col (1e-6 relative) and the rows' new parameters
(1 bf16 ulp).  Factored off: the same blocks through oracle.block_step
(indices, magnitude bit-exact, vmean 1e-6, parameters 1 ulp).  The
128-element q/k-norms and the final norm go whole through oracle.block_step.
Periods of a transposed k view and a q-norm are checked against
oracle.find_period on their step-1 grads (in the view's logical order).
"""
import sys

import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import BlockProbe, FactoredProbe, assert_within_ulp

pytestmark = pytest.mark.gpu

LR, BETAS, EPS, WD = 6e-5, (0.9, 0.999), 1e-8, 0.01
WARMUP = 2

PROBED_2D = {
    "model.embed_tokens.weight": "embed",
    "model.layers.0.self_attn.q_proj.weight": "q",
    "model.layers.0.self_attn.o_proj.weight": "o",
    "model.layers.0.mlp.up_proj.weight": "up",
    "model.layers.1.self_attn.k_proj.weight": "k (view)",
    "model.layers.2.mlp.gate_proj.weight": "gate (view)",
    "model.layers.5.self_attn.o_proj.weight": "o (view)",
    "model.layers.6.mlp.down_proj.weight": "down (view)",
}
WHOLE_1D = ("model.layers.0.self_attn.q_norm.weight", "model.layers.3.self_attn.k_norm.weight", "model.norm.weight")
PERIOD_CHECKED = ("model.layers.1.self_attn.k_proj.weight", "model.layers.0.self_attn.q_norm.weight")


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
    if free < 40 * (1 << 30):
        pytest.skip("needs about 40 GiB of free device memory")
    return torch.device("cuda", 0)


@pytest.mark.parametrize("factored", [True, False])
def test_qwen3_4b_set_local_parity(dev, factored):
    import bench
    from gefen import Gefen
    params = bench.make_qwen_params(torch, dev)
    byname = dict(params)
    views = {n for n, p in params if not p.is_contiguous()}
    assert len(views) == 25
    for n, cls in PROBED_2D.items():
        assert (n in views) == ("view" in cls), n
    opt = Gefen(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, factored_v_2d=factored)
    step1 = {}
    for w in range(WARMUP):
        bench.fill_qwen_grads(torch, params, w, dev)
        if w == 0:
            step1 = {n: _f(byname[n].grad).reshape(-1) for n in PERIOD_CHECKED}
        opt.step()
    torch.cuda.synchronize()
    _say("qwen3-4b factored=%s: %d warm-up steps done" % (factored, WARMUP))
    for n, g in step1.items():
        shape = tuple(byname[n].shape)
        assert opt.state[byname[n]]["automatic_period"] == orc.find_period(g, shape), n
    cb = opt._gefen_codebook.cpu().numpy()

    bench.fill_qwen_grads(torch, params, WARMUP, dev)
    probes = []
    for n, cls in PROBED_2D.items():
        p = byname[n]
        st = opt.state[p]
        P = st["automatic_period"]
        R, C = p.shape
        nb = p.numel() // P
        tag = "%s (%s, P=%d)" % (cls, n, P)
        if factored:
            rows = [0, 1, R // 2, (nb // 2) * P // C, R - 1]
            probe = FactoredProbe(tag, p, P, rows, [0, 7, C // 2, C - 1], [0, nb // 2, nb - 1])
        else:
            probe = BlockProbe(tag, p, P, [0, nb // 2, nb - 1])
        probe.capture(st)
        probes.append(probe)
    whole = {}
    for n in WHOLE_1D:
        p, st = byname[n], opt.state[byname[n]]
        whole[n] = (_f(p), _f(p.grad), st["m_codebook"].cpu().numpy().reshape(-1),
                    st["m_magnitude"].cpu().numpy().reshape(-1), st["vmean"].cpu().numpy().reshape(-1))
    opt.step()
    torch.cuda.synchronize()
    step = WARMUP + 1
    _say("qwen3-4b factored=%s: checked step %d done" % (factored, step))
    for probe in probes:
        probe.verify(opt.state[probe.p], cb, step=step, beta1=BETAS[0], beta2=BETAS[1], lr=LR, eps=EPS, wd=WD)
        _say("  %s ok" % probe.name)
    bc1, bc2 = 1 - BETAS[0] ** step, 1 - BETAS[1] ** step
    for n, (p0, g0, i0, m0, v0) in whole.items():
        p, st = byname[n], opt.state[byname[n]]
        P = st["automatic_period"]
        p1, i1, m1, v1 = orc.block_step(p0, g0, i0, m0, v0, P, cb, orc.BF16, beta1=BETAS[0], beta2=BETAS[1],
                                        lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=WD)
        np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), i1, err_msg=n + " indices")
        np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), m1, err_msg=n + " magnitudes")
        np.testing.assert_allclose(st["vmean"].cpu().numpy().reshape(-1), v1, rtol=1e-6, err_msg=n + " vmean")
        assert_within_ulp(_f(p), p1, orc.BF16, n + " p", atol=1e-6 * LR)
        _say("  %s (P=%d) ok" % (n, P))
    del opt
    for _, p in params:
        p.grad = None
    torch.cuda.empty_cache()
