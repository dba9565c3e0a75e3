"""BASELINE config 3 in miniature, end to end through the optimizer class:
a Qwen3-shaped parameter set (GQA q / k / v / o, gate / up / down, 128-element
q/k-norm vectors, two norms per layer, a tied embedding, a final norm) with
some 2D parameters passed as transposed views (storage [C, R] seen as .t()),
Student-t (nu = 3) grads scaled by 1e-3, factored_v_2d on and off.

Step 1 runs the real period search and codebook learning on the GPU; both
must equal the oracle's (periods: partitioning.py:237-313; codebook:
gefen.py:417-517).  Then every step's indices and magnitudes must be
bit-exact against the oracle's decomposed step, v statistics within 1e-6 and
parameters within one bf16 ulp.  The full-size set (4.0e9 parameters) is the
bench's `--workload qwen`.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from local_checks import assert_within_ulp

pytestmark = pytest.mark.gpu

H, Q, KV, FF, HD, V = 320, 512, 128, 1216, 128, 1024
LR, BETAS, EPS, WD = 6e-5, (0.9, 0.999), 1e-8, 0.01
TRANSPOSED = {"model.layers.0.self_attn.o_proj.weight", "model.layers.1.mlp.down_proj.weight"}


def qwen_shapes(layers=2, hidden=H, q=Q, kv=KV, ff=FF, head_dim=HD, vocab=V):
    shapes = [("model.embed_tokens.weight", (vocab, hidden))]
    for i in range(layers):
        pre = "model.layers.%d." % i
        shapes += [(pre + "self_attn.q_proj.weight", (q, hidden)), (pre + "self_attn.k_proj.weight", (kv, hidden)),
                   (pre + "self_attn.v_proj.weight", (kv, hidden)), (pre + "self_attn.o_proj.weight", (hidden, q)),
                   (pre + "self_attn.q_norm.weight", (head_dim,)), (pre + "self_attn.k_norm.weight", (head_dim,)),
                   (pre + "mlp.gate_proj.weight", (ff, hidden)), (pre + "mlp.up_proj.weight", (ff, hidden)),
                   (pre + "mlp.down_proj.weight", (hidden, ff)), (pre + "input_layernorm.weight", (hidden,)),
                   (pre + "post_attention_layernorm.weight", (hidden,))]
    shapes.append(("model.norm.weight", (hidden,)))
    return shapes


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _student_t(shape, rng):
    return (rng.standard_t(3, size=shape) * 1e-3).astype(np.float32)


@pytest.mark.parametrize("factored", [True, False])
def test_qwen_shaped_set_matches_oracle(dev, factored):
    from gefen import Gefen
    rng = np.random.default_rng(42)
    shapes = qwen_shapes()
    params, ref = [], {}
    for name, shape in shapes:
        p0 = orc.round_dtype((rng.standard_normal(shape) * 0.02).astype(np.float32), orc.BF16)
        if name in TRANSPOSED:
            storage = torch.from_numpy(np.ascontiguousarray(p0.T)).to(torch.bfloat16).to(dev)
            p = torch.nn.Parameter(storage.t())
            assert not p.is_contiguous()
        else:
            p = torch.nn.Parameter(torch.from_numpy(p0).to(torch.bfloat16).to(dev))
        params.append((name, p))
        ref[name] = {"p": p0.copy()}
    opt = Gefen(params, lr=LR, betas=BETAS, eps=EPS, weight_decay=WD, factored_v_2d=factored)
    cb = None
    for step in range(1, 4):
        grads = {}
        for name, p in params:
            g = orc.round_dtype(_student_t(tuple(p.shape), rng), orc.BF16)
            grads[name] = g
            gt = torch.from_numpy(g).to(torch.bfloat16).to(dev)
            p.grad = gt.t().contiguous().t() if name in TRANSPOSED else gt
        opt.step()
        torch.cuda.synchronize()
        if step == 1:
            # periods and codebook of the GPU step 1 against the oracle
            for name, p in params:
                per = int(opt.state[p]["automatic_period"])
                numel = p.numel()
                want = 1 if numel == 1 else orc.find_period(grads[name].reshape(-1), tuple(p.shape))
                assert per == want, "%s: period %d, oracle %d" % (name, per, want)
                ref[name]["per"] = per
            cb = orc.learn_codebook([(grads[n].reshape(-1), ref[n]["per"]) for n, _ in params])
            np.testing.assert_array_equal(opt._gefen_codebook.cpu().numpy(), cb, err_msg="codebook")
        bc1, bc2 = 1 - BETAS[0] ** step, 1 - BETAS[1] ** step
        for name, p in params:
            r = ref[name]
            g = grads[name]
            per = r["per"]
            st = opt.state[p]
            is_fact = factored and p.ndim == 2
            if step == 1:
                nb = p.numel() // per
                r["idx"] = np.zeros(p.numel(), np.uint8)
                r["mag"] = np.zeros(nb, np.float32)
                if is_fact:
                    r["vr"] = np.zeros(p.shape[0], np.float32)
                    r["vc"] = np.zeros(p.shape[1], np.float32)
                else:
                    r["vm"] = np.zeros(nb, np.float32)
            if is_fact:
                r["p"], r["idx"], r["mag"], r["vr"], r["vc"] = orc.factored_step(
                    r["p"], g, r["idx"], r["mag"], r["vr"], r["vc"], per, cb, orc.BF16, beta1=BETAS[0],
                    beta2=BETAS[1], lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=WD)
            else:
                r["p"], r["idx"], r["mag"], r["vm"] = orc.block_step(
                    r["p"], g, r["idx"], r["mag"], r["vm"], per, cb, orc.BF16, beta1=BETAS[0], beta2=BETAS[1],
                    lr=LR, eps=EPS, bc1=bc1, bc2=bc2, wd=WD)
            tag = "factored=%s step %d %s" % (factored, step, name)
            np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), r["idx"], err_msg=tag)
            np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), r["mag"], err_msg=tag)
            if is_fact:
                np.testing.assert_allclose(st["v_row"].cpu().numpy(), r["vr"], rtol=1e-6, err_msg=tag)
                np.testing.assert_allclose(st["v_col"].cpu().numpy(), r["vc"], rtol=1e-6, err_msg=tag)
            else:
                np.testing.assert_allclose(st["vmean"].cpu().numpy().reshape(-1), r["vm"], rtol=1e-6, err_msg=tag)
            got = p.detach().float().cpu().numpy()
            assert_within_ulp(got, r["p"], orc.BF16, tag, atol=1e-6 * LR)
            r["p"] = got  # continue from the GPU's parameters (p may differ by an ulp)
