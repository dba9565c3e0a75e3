"""torch.compile on the GPU: the gefen:: custom ops give the eager kernels'
results bit for bit, the period-variance entry matches a float64 restatement,
and a compiled capturable Gefen.step follows the eager trajectory exactly
(the reference's tests/test_capturable.py:520-565 pins the same parity; graph
breaks at host-side helpers are allowed by design there too)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from gefen.kernels import _native
    _native.load()
    return torch.device("cuda", 0)


def _say(msg):
    print(msg, flush=True)


def _codebook(dev):
    import os
    gold = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "learn.npz")
    return torch.from_numpy(np.load(gold)["cb"]).to(dev)


def _state(dev, rows, cols, period, seed):
    gen = torch.Generator().manual_seed(seed)
    nb = rows * cols // period
    return dict(p=(torch.randn(rows, cols, generator=gen) * 0.02).to(torch.bfloat16).to(dev),
                m_sign=torch.zeros(nb, period, dtype=torch.uint8, device=dev),
                m_magnitude=torch.zeros(nb, 1, device=dev),
                v_row=torch.zeros(rows, device=dev), v_col=torch.zeros(cols, device=dev))


def test_compiled_factored_op_matches_eager(dev):
    from gefen.kernels import automatic_gefen_fused as fused
    rows, cols, period = 96, 1024, 8192
    cb = _codebook(dev)
    lut = fused._codebook_search_lut(cb)
    a, b = _state(dev, rows, cols, period, 1), _state(dev, rows, cols, period, 1)
    gen = torch.Generator().manual_seed(2)

    def step(st, g, scalars):
        fused.gefen_factored_update_cuda(st["p"], g, st["m_sign"], st["m_magnitude"], st["v_row"], st["v_col"],
                                         cb, cols, 0.9, 0.999, 0.0, 1e-8, 0.0, 0.0, 0.0,
                                         step_scalars=scalars, codebook_lut=lut)

    torch._dynamo.reset()
    compiled = torch.compile(step, backend="aot_eager", fullgraph=True)
    for s in range(1, 4):
        g = (torch.randn(rows * cols // period, period, generator=gen) * 1e-3).to(torch.bfloat16).to(dev)
        bc1, bc2 = 1 - 0.9 ** s, 1 - 0.999 ** s
        scalars = torch.tensor([6e-5, 1 / bc2, 1 / bc1, 1 - 6e-5 * 0.01], dtype=torch.float32, device=dev)
        step(a, g, scalars)
        compiled(b, g, scalars)
        torch.cuda.synchronize()
        for k in a:
            assert torch.equal(a[k], b[k]), (s, k)
        _say("compiled factored step %d equal" % s)
    torch._dynamo.reset()


def test_compiled_momentum_op_matches_eager(dev):
    from gefen.kernels import automatic_gefen_fused as fused
    n, period = 4096 * 16, 4096
    cb = _codebook(dev)
    lut = fused._codebook_search_lut(cb)
    nb = n // period
    outs = []
    for mode in ("eager", "compiled"):
        idx = torch.zeros(nb, period, dtype=torch.uint8, device=dev)
        mag = torch.zeros(nb, 1, device=dev)
        mom = torch.empty(nb, period, dtype=torch.bfloat16, device=dev)
        gen = torch.Generator().manual_seed(5)

        def step(g):
            fused.gefen_quantized_momentum_update_cuda(g, idx, mag, cb, mom, 0.95, codebook_lut=lut,
                                                       nesterov=True)

        fn = step if mode == "eager" else torch.compile(step, backend="aot_eager", fullgraph=True)
        for _ in range(3):
            fn((torch.randn(nb, period, generator=gen) * 1e-3).to(torch.bfloat16).to(dev))
        torch.cuda.synchronize()
        outs.append((idx.clone(), mag.clone(), mom.clone()))
    for x, y in zip(*outs):
        assert torch.equal(x, y)
    torch._dynamo.reset()


def _variance_ref(x, period, squared):
    x32 = x.astype(np.float32)
    v = x32.astype(np.float64) if squared else (x32 * x32).astype(np.float64)  # fp32 square, then float64
    blocks = v.reshape(-1, period)
    return float(np.sqrt(np.mean(np.var(blocks, axis=1))))


@pytest.mark.parametrize("period", [1, 48, 1024, 65536 * 3])
@pytest.mark.parametrize("squared", [False, True])
def test_average_within_block_variance_matches_float64(dev, period, squared):
    from gefen.kernels.period_variance import average_within_block_variance_cuda_kernel
    gen = torch.Generator().manual_seed(period)
    n = period * max(1, (1 << 20) // period)
    x = torch.randn(n, generator=gen) * 1e-2
    if squared:
        x = x * x
    got = average_within_block_variance_cuda_kernel(x.to(dev), period, input_is_squared=squared)
    ref = _variance_ref(x.numpy(), period, squared)
    assert got == pytest.approx(ref, rel=1e-12, abs=1e-30), (got, ref)
    op = torch.ops.gefen.average_within_block_variance_cuda(x.to(dev), period, squared)
    assert op.dim() == 0 and op.device == dev and float(op) == pytest.approx(got, rel=1e-7)


def test_average_within_block_variance_checks(dev):
    from gefen.kernels.period_variance import average_within_block_variance_cuda_kernel
    with pytest.raises(ValueError):
        average_within_block_variance_cuda_kernel(torch.ones(10), 5, input_is_squared=True)
    with pytest.raises(ValueError):
        average_within_block_variance_cuda_kernel(torch.ones(10, device=dev), 3, input_is_squared=True)
    with pytest.raises(ValueError):
        average_within_block_variance_cuda_kernel(torch.ones(10, device=dev), 0, input_is_squared=True)
    with pytest.raises(TypeError):
        average_within_block_variance_cuda_kernel([1.0], 1, input_is_squared=True)


def test_compiled_capturable_gefen_step_matches_eager(dev):
    from gefen import Gefen
    specs = [("w", (64, 1024)), ("v", (128, 512)), ("norm", (1024,))]
    steps, warmup = 6, 2

    def run(compiled):
        gen = torch.Generator().manual_seed(11)
        params = [(n, torch.nn.Parameter((torch.randn(*s, generator=gen) * 0.02).to(torch.bfloat16).to(dev)))
                  for n, s in specs]
        opt = Gefen(params, lr=1e-3, weight_decay=0.01, capturable=True)
        fn = torch.compile(opt.step, backend="eager") if compiled else opt.step
        ggen = torch.Generator().manual_seed(12)
        for i in range(steps):
            for _, p in params:
                p.grad = (torch.randn(p.shape, generator=ggen) * 1e-3).to(torch.bfloat16).to(dev)
            (fn if i >= warmup else opt.step)()
        torch.cuda.synchronize()
        return [p.detach().clone() for _, p in params], opt.state_dict()["gefen_global_step"]

    torch._dynamo.reset()
    ref, ref_step = run(False)
    got, got_step = run(True)
    torch._dynamo.reset()
    assert ref_step == got_step == steps
    for a, b in zip(ref, got):
        assert torch.equal(a, b)
