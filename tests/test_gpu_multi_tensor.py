"""gefenx_multi_tensor_step against one call per parameter, and against
the oracle.

Both paths run the same phase code on the same per-parameter workgroup
partition, so the multi-tensor launcher must reproduce the per-parameter
entry points exactly: indices, magnitudes, second-moment state and params
bit-identical (the block path's float64 per-block sums are reduced with
atomics whose order may differ, hence the 1-ulp allowance on vmean and the
params of block-path tensors).  Every tensor of the launcher's run is also
checked against the oracle's decomposed step after every step
(tests/local_checks.StepTracker: step-1 periods and codebook equal to the
oracle's, indices and magnitudes bit-exact, v within 1e-6, params within
1 ulp / 1e-6 relative).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from local_checks import StepTracker

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _make(shapes, dtypes, dev, seed):
    gen = torch.Generator().manual_seed(seed)
    out = []
    for i, (shape, dt) in enumerate(zip(shapes, dtypes)):
        if isinstance(shape, tuple) and len(shape) == 3 and shape[2] == "T":
            base = (torch.randn(shape[1], shape[0], generator=gen) * 0.02).to(dt)
            out.append(("t%d" % i, base, True))
        else:
            out.append(("t%d" % i, (torch.randn(*shape, generator=gen) * 0.02).to(dt), False))
    return out


def _params(init, dev):
    ps = []
    for name, t, transposed in init:
        if transposed:
            base = t.to(dev).clone()
            p = torch.nn.Parameter(base.t())  # non-contiguous view
        else:
            p = torch.nn.Parameter(t.to(dev).clone())
        ps.append((name, p))
    return ps


def _grads(params, step, seed):
    gen = torch.Generator().manual_seed(seed * 1000 + step)
    for i, (_, p) in enumerate(params):
        sigma = 10.0 ** (-4 + 2 * ((i * 7 + step) % 5) / 4)
        g = (torch.randn(*p.shape, generator=gen) * sigma).to(p.dtype).to(p.device)
        if i % 3 == 1 and p.ndim == 2:
            g = g.t().contiguous().t()  # strided grad for some factored tensors
        p.grad = g


def _run(dev, shapes, dtypes, steps=4, seed=0, **kw):
    from gefen import Gefen
    init = _make(shapes, dtypes, dev, seed)
    pa, pb = _params(init, dev), _params(init, dev)
    oa = Gefen(pa, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, **kw)
    ob = Gefen(pb, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, **kw)
    oa._multi_tensor = True
    ob._multi_tensor = False
    track = StepTracker(1e-3, 0.01, kw.get("factored_v_2d", True))
    for name, a in pa:
        if a.numel():
            track.track(name, a)
    for s in range(steps):
        _grads(pa, s, seed)
        _grads(pb, s, seed)
        grads = {name: a.grad.float().cpu().numpy().copy() for name, a in pa}
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        if s == 0:
            track.learn(oa, pa, grads)
        for name, a in pa:
            track.step(name, grads[name])
            track.check(oa, name, a, "launcher vs oracle")
        for (name, a), (_, b) in zip(pa, pb):
            sa, sb = oa.state[a], ob.state[b]
            tag = "%s %s %s step %d" % (name, tuple(a.shape), a.dtype, s + 1)
            assert sa["automatic_period"] == sb["automatic_period"], tag
            assert torch.equal(sa["m_codebook"], sb["m_codebook"]), tag
            assert torch.equal(sa["m_magnitude"], sb["m_magnitude"]), tag
            if "v_row" in sa:
                assert torch.equal(sa["v_row"], sb["v_row"]), tag
                assert torch.equal(sa["v_col"], sb["v_col"]), tag
                assert torch.equal(a.detach(), b.detach()), tag
            else:
                torch.testing.assert_close(sa["vmean"], sb["vmean"], rtol=2.0 ** -23, atol=0.0, msg=tag)
                torch.testing.assert_close(a.detach().float(), b.detach().float(),
                                           rtol=2.0 ** -7, atol=1e-9, msg=tag)
    return oa, pa


def test_mixed_set_matches_per_parameter(dev):
    shapes = [(64, 96), (40, 72), (32, 64), (4096,), (999,), (7, 4100), (300, 24), (96, 64, "T"),
              (1024, 2048), (3000,), (1,), (48, 128)]
    dtypes = [torch.bfloat16, torch.float32, torch.float16, torch.bfloat16, torch.float32,
              torch.bfloat16, torch.float32, torch.bfloat16, torch.bfloat16, torch.float16,
              torch.float32, torch.bfloat16]
    _run(dev, shapes, dtypes)


def test_block_path_for_2d_matches_per_parameter(dev):
    # indices 1 and 4 get strided grads: transposed views stepped in place by
    # the launcher; index 5 is a view with a contiguous grad (copy route)
    shapes = [(64, 96), (200, 136, "T"), (4096,), (1000,), (328, 200, "T"), (96, 64, "T"), (40, 72)]
    dtypes = [torch.bfloat16, torch.bfloat16, torch.bfloat16, torch.float32, torch.float32, torch.float16,
              torch.float32]
    _run(dev, shapes, dtypes, factored_v_2d=False)


def test_many_small_tensors(dev):
    # a few hundred norm-sized vectors: the workgroup -> tensor lookup spans
    # many segments in each launch
    shapes = [(512,)] * 150 + [(64, 64)] * 150
    dtypes = [torch.bfloat16] * 300
    _run(dev, shapes, dtypes, steps=2, seed=3)


def test_empty_and_gradless_params_are_skipped(dev):
    from gefen import Gefen
    a = torch.nn.Parameter(torch.randn(64, 96, device=dev, dtype=torch.bfloat16) * 0.02)
    e = torch.nn.Parameter(torch.empty(0, 5, device=dev, dtype=torch.bfloat16))
    n = torch.nn.Parameter(torch.randn(32, device=dev, dtype=torch.bfloat16))
    opt = Gefen([a, e, n], lr=1e-3)
    a.grad = torch.randn_like(a) * 1e-3
    e.grad = torch.empty_like(e)
    before = n.detach().clone()
    opt.step()
    torch.cuda.synchronize()
    assert torch.equal(n.detach(), before)
    assert "m_codebook" in opt.state[a]


@pytest.mark.parametrize("pipeline", ["1", "0"])
def test_cohorts_match_one_launch_set(dev, monkeypatch, pipeline):
    """Cohorts (GEFENX_COHORT_ELEMS): several launch sets per step, with the
    stats of later cohorts on the side stream while earlier cohorts apply
    (GEFENX_PIPELINE=1) or all on the caller's stream; results equal the
    single-cohort step bit for bit, and work enqueued on the caller's stream
    afterwards sees the whole step."""
    from gefen import Gefen
    shapes = [(64, 96), (1024, 2048), (4096,), (300, 24), (96, 64, "T"), (512, 512), (999,), (128, 640)]
    dtypes = [torch.bfloat16, torch.bfloat16, torch.float32, torch.float32, torch.bfloat16, torch.float16,
              torch.bfloat16, torch.bfloat16]
    init = _make(shapes, dtypes, dev, 7)
    pa, pb = _params(init, dev), _params(init, dev)
    oa = Gefen(pa, lr=1e-3, weight_decay=0.01)
    ob = Gefen(pb, lr=1e-3, weight_decay=0.01)
    for s in range(3):
        _grads(pa, s, 7)
        _grads(pb, s, 7)
        monkeypatch.setenv("GEFENX_COHORT_ELEMS", "300000")  # several cohorts
        monkeypatch.setenv("GEFENX_PIPELINE", pipeline)
        oa.step()
        # read back right after the step on the caller's stream (no device sync)
        snap = [a.detach().clone() for _, a in pa]
        monkeypatch.delenv("GEFENX_COHORT_ELEMS")
        monkeypatch.delenv("GEFENX_PIPELINE")
        ob.step()
        torch.cuda.synchronize()
        for (name, a), (_, b), sa_p in zip(pa, pb, snap):
            tag = "%s %s step %d pipeline %s" % (name, tuple(a.shape), s + 1, pipeline)
            sa, sb = oa.state[a], ob.state[b]
            assert torch.equal(sa["m_codebook"], sb["m_codebook"]), tag
            assert torch.equal(sa["m_magnitude"], sb["m_magnitude"]), tag
            assert torch.equal(a.detach(), b.detach()), tag
            assert torch.equal(sa_p, b.detach()), tag
