"""Device mobility of the optimizer state on MI355X (CPU offload).

A CPU-offload trainer pages parameters (and often the optimizer state) off
the GPU between steps.  Gefen moves a parameter's state to the parameter's
device at its next step (reference gefen.py:1897-1927); the step then runs
on the HIP kernels as usual.  The continued trajectory is checked against
the reference's own: tests/golden/ckpt_<case>.pt is the reference's
state_dict after three CPU steps and ckpt_<case>.npz the states the
reference reaches from it (indices and magnitudes bit-exact, second moments
within 1e-6, parameters within one bf16 ulp).

``fused=False`` is the reference's decomposed step; it computes the same
arithmetic, so it runs on the same kernels with bit-identical results.
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
STATE_KEYS = ("m_codebook", "m_magnitude", "v_row", "v_col", "vmean")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _tensor_devices(opt, p):
    return {k: v.device for k, v in opt.state[p].items() if torch.is_tensor(v) and not k.startswith("_")}


@pytest.mark.parametrize("case", ["fact_bf16", "block_bf16"])
@pytest.mark.parametrize("fused", [True, False])
def test_state_paged_to_host_follows_reference(dev, case, fused):
    """Before every continued step the parameter is paged GPU -> host -> GPU
    and its state is left on the host; the step must bring the state back
    and land on the reference's next state."""
    from gefen import Gefen
    print("colocate", case, "fused", fused, flush=True)
    sd = torch.load(os.path.join(GOLD, "ckpt_%s.pt" % case), weights_only=True)
    ref = np.load(os.path.join(GOLD, "ckpt_%s.npz" % case))
    pre, steps = int(ref["pre"]), int(ref["steps"])
    names = ("w", "b")
    params = [(n, torch.nn.Parameter(torch.from_numpy(ref["p%d_%s" % (pre, n)]).to(torch.bfloat16).to(dev)))
              for n in names]
    opt = Gefen(params, lr=6e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=float(ref["wd"]),
                factored_v_2d=bool(ref["factored"]), fused=fused)
    opt.load_state_dict(copy.deepcopy(sd))
    for s in range(pre + 1, steps + 1):
        for n, p in params:
            st = opt.state[p]
            for k in list(st):
                if torch.is_tensor(st[k]):
                    st[k] = st[k].cpu()  # the state stranded on the host
            p.data = p.data.cpu()
            p.data = p.data.to(dev)
            p.grad = torch.from_numpy(ref["g%d_%s" % (s, n)]).to(torch.bfloat16).to(dev)
        opt.step()
        torch.cuda.synchronize()
        for n, p in params:
            st = opt.state[p]
            tag = "%s step %d %s" % (case, s, n)
            assert set(d.type for d in _tensor_devices(opt, p).values()) == {"cuda"}, tag
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


def _run(dev, fused, page_every=None, n_params=6, steps=5, factored=True):
    """Several same-shape tensors (one multi-tensor batch); with page_every,
    the state of every other tensor is sent to the host before each step."""
    from gefen import Gefen
    gen = torch.Generator().manual_seed(5)
    ps = [("w%d" % i, torch.nn.Parameter((torch.randn(48, 64, generator=gen) * 0.02).to(torch.bfloat16).to(dev)))
          for i in range(n_params)]
    opt = Gefen(ps, lr=1e-3, weight_decay=0.01, fused=fused, factored_v_2d=factored)
    for s in range(steps):
        for i, (_, p) in enumerate(ps):
            p.grad = (torch.randn(48, 64, generator=gen) * 1e-3).to(torch.bfloat16).to(dev)
            if page_every and s > 0 and i % page_every == 0:
                st = opt.state[p]
                for k in STATE_KEYS:
                    if k in st:
                        st[k] = st[k].cpu()
        opt.step()
    torch.cuda.synchronize()
    return ps, opt


@pytest.mark.parametrize("factored", [True, False])
def test_batch_with_stranded_state_equals_resident_run(dev, factored):
    ps_a, a = _run(dev, True, factored=factored)
    ps_b, b = _run(dev, True, page_every=2, factored=factored)
    for (n, pa), (_, pb) in zip(ps_a, ps_b):
        assert set(d.type for d in _tensor_devices(b, pb).values()) == {"cuda"}, n
        for k in STATE_KEYS:
            if k in a.state[pa]:
                assert torch.equal(a.state[pa][k], b.state[pb][k]), (n, k)
        assert torch.equal(pa, pb), n


def test_fused_false_is_the_same_step(dev):
    ps_a, a = _run(dev, True)
    ps_b, b = _run(dev, False)
    assert b.fused is False
    for (n, pa), (_, pb) in zip(ps_a, ps_b):
        for k in STATE_KEYS:
            if k in a.state[pa]:
                assert torch.equal(a.state[pa][k], b.state[pb][k]), (n, k)
        assert torch.equal(pa, pb), n


def test_capturable_host_parameter_is_refused_before_any_mutation(dev):
    """Host parameters are stepped through pinned staging (tests/
    test_gpu_host_resident.py), but not under capturable=True: a graph
    cannot record host memory."""
    from gefen import Gefen
    p = torch.nn.Parameter(torch.randn(16, 16))
    opt = Gefen([("w", p)], lr=1e-2, capturable=True)
    p.grad = torch.randn(16, 16) * 0.1
    with pytest.raises(RuntimeError, match="capturable=True steps HIP device parameters only"):
        opt.step()
    assert opt._gefen_codebook is None
    assert "automatic_period" not in opt.state.get(p, {})


def test_grad_param_device_mismatch_is_refused_before_any_mutation(dev):
    from gefen import Gefen
    p = torch.nn.Parameter(torch.randn(8, 8).to(dev))
    opt = Gefen([("w", p)], lr=1e-2)
    p.grad = torch.randn(8, 8, device=dev) * 0.1
    p.data = p.data.cpu()  # paged after its gradient was set
    with pytest.raises(RuntimeError, match="same device"):
        opt.step()
    assert opt._gefen_codebook is None
    assert "automatic_period" not in opt.state.get(p, {})
    # back on the GPU with its gradient: the step runs and learns the codebook
    p.data = p.data.to(dev)
    opt.step()
    assert opt._gefen_codebook is not None and torch.isfinite(p).all()
