"""Host-resident parameters (CPU offload) stepped on MI355X.

Mirrors the reference's tests/test_cpu_resident_step.py: a parameter paged
CPU -> GPU -> CPU between steps, a batch of same-shape parameters paged
together, a checkpoint saved on the GPU and resumed on host-resident
parameters, a grad/param device split refused before the codebook is learned,
a tensor lr on the GPU while the parameter is on the host, and resume after
paging.  The reference steps host parameters with its decomposed CPU step;
here they are stepped on the GPU through pinned staging, and every step is
checked against the oracle (the reference's decomposed step): requantised
indices and magnitudes bit-exact, v_row / v_col / vmean within 1e-6, and
parameters within 1 ulp (bf16) or 1e-6 relative (fp32).  Step 1's period
search and codebook must equal the oracle's.  After each step every state
tensor must be on the parameter's device, as the reference requires.
"""
import copy
import io

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import oracle as orc
from local_checks import StepTracker, assert_within_ulp

pytestmark = pytest.mark.gpu



@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _state_devices(opt, p):
    """Devices of every tensor-valued state entry of p (all keys, as the
    reference's test checks them)."""
    return {k: v.device for k, v in opt.state[p].items() if torch.is_tensor(v)}


def _run_schedule(named, opt, orc_, schedule, gen, scale, tag, lr_of=None):
    """Page every parameter to the scheduled device, set fresh grads, step,
    then check the state's devices and the oracle."""
    for k, device in enumerate(schedule):
        grads = {}
        for name, p in named:
            p.data = p.data.to(device)
            g = (torch.randn(p.shape, generator=gen) * scale).to(p.dtype)
            grads[name] = g.float().numpy().copy()
            p.grad = g.to(device)
        print("%s: step %d on %s" % (tag, k + 1, device), flush=True)
        opt.step()
        opt.zero_grad(set_to_none=True)
        torch.cuda.synchronize()
        if orc_.cb is None:
            orc_.learn(opt, named, grads)
        lr = None if lr_of is None else lr_of()
        for name, p in named:
            assert p.device.type == device.type
            devs = _state_devices(opt, p)
            assert devs and set(d.type for d in devs.values()) == {device.type}, (tag, name, devs)
            orc_.step(name, grads[name], lr=lr)
            orc_.check(opt, name, p, tag, lr=lr)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("factored", [True, False])
def test_param_paged_cpu_gpu_cpu_across_steps(dev, factored, dtype):
    """Reference tests/test_cpu_resident_step.py:128-157."""
    from gefen import Gefen
    torch.manual_seed(0)
    p = nn.Parameter(torch.randn(16, 16).to(dtype))
    named = [("w", p)]
    opt = Gefen(named, lr=1e-2, fused=False, factored_v_2d=factored)
    track = StepTracker(1e-2, 0.0, factored)
    track.track("w", p)
    before = p.detach().cpu().clone()
    cpu = torch.device("cpu")
    _run_schedule(named, opt, track, [cpu, dev, cpu], torch.Generator().manual_seed(3), 0.1,
                  "paged factored=%s %s" % (factored, dtype))
    assert opt._gefen_codebook.device.type == "cpu"  # learned from the host-resident gradient
    assert p.device.type == "cpu" and torch.isfinite(p).all() and not torch.equal(before, p.detach())


def test_batched_group_paged_cpu_gpu_cpu(dev):
    """Reference tests/test_cpu_resident_step.py:160-186: six same-shape
    parameters, paged together."""
    from gefen import Gefen
    torch.manual_seed(0)
    named = [("w%d" % i, nn.Parameter(torch.randn(8, 12))) for i in range(6)]
    opt = Gefen(named, lr=1e-2, fused=False, factored_v_2d=False)
    track = StepTracker(1e-2, 0.0, False)
    for n, p in named:
        track.track(n, p)
    cpu = torch.device("cpu")
    _run_schedule(named, opt, track, [cpu, dev, dev, cpu], torch.Generator().manual_seed(5), 0.1, "batched")
    assert all(p.device.type == "cpu" for _, p in named)


def test_grad_on_other_device_than_param_is_refused(dev):
    """Reference tests/test_cpu_resident_step.py:189-205."""
    from gefen import Gefen
    p = nn.Parameter(torch.randn(8, 8).to(dev))
    opt = Gefen([("w", p)], lr=1e-2, fused=False)
    p.grad = torch.randn(8, 8, device=dev) * 0.1
    p.data = p.data.cpu()
    assert p.device.type == "cpu" and p.grad.device.type == "cuda"
    with pytest.raises(RuntimeError, match="same device"):
        opt.step()


@pytest.mark.parametrize("factored", [True, False])
def test_checkpoint_saved_on_gpu_loads_and_steps_on_host(dev, factored):
    """Reference tests/test_cpu_resident_step.py:207-258: save on the GPU,
    torch.load(map_location='cpu'), load into an optimizer of host
    parameters, step: state and codebook on the host, the step the
    oracle's from the checkpointed state."""
    from gefen import Gefen
    torch.manual_seed(0)
    model_gpu = nn.Sequential(nn.Linear(32, 48), nn.Tanh(), nn.Linear(48, 16)).to(dev)
    names = [n for n, _ in model_gpu.named_parameters()]
    opt_gpu = Gefen(list(model_gpu.named_parameters()), lr=1e-3, fused=False, factored_v_2d=factored)
    gen = torch.Generator().manual_seed(11)
    for _ in range(3):
        for p in model_gpu.parameters():
            p.grad = (torch.randn(p.shape, generator=gen) * 1e-2).to(dev)
        opt_gpu.step()
        opt_gpu.zero_grad()
    buf = io.BytesIO()
    torch.save(opt_gpu.state_dict(), buf)
    buf.seek(0)
    cpu_state = torch.load(buf, map_location="cpu", weights_only=True)

    model_cpu = nn.Sequential(nn.Linear(32, 48), nn.Tanh(), nn.Linear(48, 16))
    with torch.no_grad():
        for pc, pg in zip(model_cpu.parameters(), model_gpu.parameters()):
            pc.copy_(pg.cpu())
    opt_cpu = Gefen(list(model_cpu.named_parameters()), lr=1e-3, fused=False, factored_v_2d=factored)
    opt_cpu.load_state_dict(cpu_state)
    assert opt_cpu._gefen_codebook.device.type == "cpu"
    for p in model_cpu.parameters():
        assert set(d.type for d in _state_devices(opt_cpu, p).values()) == {"cpu"}

    # the oracle continues from the checkpointed state
    track = StepTracker(1e-3, 0.0, factored)
    track.cb = cpu_state["gefen_codebook"].float().numpy()
    np.testing.assert_array_equal(opt_gpu._gefen_codebook.cpu().numpy(), track.cb)
    for name, p in zip(names, model_cpu.parameters()):
        st = opt_cpu.state[p]
        track.track(name, p)
        r = track.ref[name]
        r["per"], r["step"] = int(st["automatic_period"]), int(st["step"])
        r["idx"] = st["m_codebook"].numpy().reshape(-1).copy()
        r["mag"] = st["m_magnitude"].numpy().reshape(-1).copy()
        if factored and p.ndim == 2:
            r["vr"], r["vc"] = st["v_row"].numpy().copy(), st["v_col"].numpy().copy()
        else:
            r["vm"] = st["vmean"].numpy().reshape(-1).copy()
    gen_cpu = torch.Generator().manual_seed(12)
    grads = {}
    for name, p in zip(names, model_cpu.parameters()):
        p.grad = torch.randn(p.shape, generator=gen_cpu) * 1e-2
        grads[name] = p.grad.numpy().copy()
    opt_cpu.step()
    for name, p in zip(names, model_cpu.parameters()):
        assert set(d.type for d in _state_devices(opt_cpu, p).values()) == {"cpu"}
        track.step(name, grads[name])
        track.check(opt_cpu, name, p, "resumed on host factored=%s" % factored)


def test_grad_param_mismatch_fails_before_codebook_mutation(dev):
    """Reference tests/test_cpu_resident_step.py:290-314."""
    from gefen import Gefen
    p = nn.Parameter(torch.randn(16, 16).to(dev))
    opt = Gefen([("w", p)], lr=1e-2, fused=False)
    p.grad = torch.randn(16, 16, device=dev) * 0.1
    p.data = p.data.cpu()
    assert opt._gefen_codebook is None
    with pytest.raises(RuntimeError, match="same device"):
        opt.step()
    assert opt._gefen_codebook is None
    assert "automatic_period" not in opt.state.get(p, {})
    # co-located on the host and retried: the codebook comes from this gradient
    track = StepTracker(1e-2, 0.0, True)
    track.track("w", p)
    g = torch.randn(16, 16) * 0.1
    p.grad = g
    opt.step()
    assert opt._gefen_codebook is not None and opt._gefen_codebook.device.type == "cpu"
    track.learn(opt, [("w", p)], {"w": g.numpy()})
    track.step("w", g.numpy())
    track.check(opt, "w", p, "mismatch retried")


@pytest.mark.parametrize("factored", [True, False])
def test_tensor_lr_survives_host_paging(dev, factored):
    """Reference tests/test_cpu_resident_step.py:316-346: a GPU tensor lr
    while the parameter steps on the host and back."""
    from gefen import Gefen
    torch.manual_seed(0)
    lr = torch.tensor(1e-2, device=dev)
    p = nn.Parameter(torch.randn(16, 24).to(dev))
    named = [("w", p)]
    opt = Gefen(named, lr=lr, fused=False, factored_v_2d=factored)
    track = StepTracker(float(lr.item()), 0.0, factored)
    track.track("w", p)
    before = p.detach().cpu().clone()
    cpu = torch.device("cpu")
    _run_schedule(named, opt, track, [dev, cpu, dev], torch.Generator().manual_seed(0), 0.1,
                  "tensor lr factored=%s" % factored)
    assert not torch.equal(before, p.detach().cpu())


@pytest.mark.parametrize("factored", [False, True])
def test_resume_after_paging_is_exact(dev, factored):
    """Reference tests/test_cpu_resident_step.py:349-398: save after the
    state moved to the host, reload, continue: bit-identical to the
    uninterrupted run, and on the oracle's trajectory."""
    from gefen import Gefen
    torch.manual_seed(0)
    init = torch.randn(16, 24)
    gen = torch.Generator().manual_seed(1)
    grads = [torch.randn(16, 24, generator=gen) * 0.1 for _ in range(3)]
    schedule = [dev, torch.device("cpu"), torch.device("cpu")]

    def run(interrupt_before):
        p = nn.Parameter(init.clone())
        opt = Gefen([("w", p)], lr=1e-2, fused=False, factored_v_2d=factored)
        for i, (g, d) in enumerate(zip(grads, schedule)):
            if i == interrupt_before:
                saved = copy.deepcopy(opt.state_dict())
                assert all(v.device.type == "cpu" for s in saved["state"].values() for v in s.values()
                           if torch.is_tensor(v))
                p = nn.Parameter(p.detach().clone())
                opt = Gefen([("w", p)], lr=1e-2, fused=False, factored_v_2d=factored)
                opt.load_state_dict(saved)
            p.data = p.data.to(d)
            p.grad = g.clone().to(d)
            opt.step()
            opt.zero_grad(set_to_none=True)
        return p.detach().cpu(), opt, p

    reference, opt, p = run(-1)
    resumed, _, _ = run(2)
    assert torch.equal(reference, resumed)
    track = StepTracker(1e-2, 0.0, factored)
    track.track("w", nn.Parameter(init.clone()))
    r = track.ref["w"]
    r["per"] = int(opt.state[p]["automatic_period"])
    assert r["per"] == orc.find_period(grads[0].numpy().reshape(-1), (16, 24))
    track.cb = opt._gefen_codebook.cpu().numpy()
    np.testing.assert_array_equal(track.cb, orc.learn_codebook([(grads[0].numpy().reshape(-1), r["per"])]))
    for g in grads:
        track.step("w", g.numpy())
    track.check(opt, "w", p, "resume factored=%s" % factored)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_host_and_device_runs_are_bit_identical(dev, dtype):
    """The reference can only promise convergence-level agreement between
    its CPU and CUDA steps (tests/test_cpu_resident_step.py:261-287); here
    both run the same kernels, so they agree bit for bit."""
    from gefen import Gefen
    torch.manual_seed(0)
    init = torch.randn(24, 32, dtype=dtype)
    grads = [torch.randn(24, 32, dtype=dtype) * 0.1 for _ in range(6)]

    def run(device):
        p = nn.Parameter(init.clone().to(device))
        opt = Gefen([("w", p)], lr=1e-2, fused=False)
        for g in grads:
            p.grad = g.clone().to(device)
            opt.step()
            opt.zero_grad(set_to_none=True)
        return p.detach().cpu(), {k: v.cpu() for k, v in opt.state[p].items() if torch.is_tensor(v)}

    p_host, st_host = run(torch.device("cpu"))
    p_dev, st_dev = run(dev)
    assert torch.equal(p_host, p_dev)
    for k in ("m_codebook", "m_magnitude", "v_row", "v_col"):
        assert torch.equal(st_host[k], st_dev[k]), k


@pytest.mark.parametrize("factored", [True, False])
def test_many_host_params_in_small_chunks_match_device_run(dev, factored, monkeypatch):
    """Chunked staging (a chunk limit far below the set's size, so most
    chunks hold one or two parameters and the two arenas alternate), mixed
    dtypes, a transposed host view (staged in logical order; its device
    twin is contiguous, since device views sum v in another order) and a
    None grad: bit-identical to the same optimizer stepping the same
    parameters on the GPU."""
    from gefen import Gefen
    monkeypatch.setenv("GEFENX_HOST_STAGING_BYTES", "8192")
    gen = torch.Generator().manual_seed(9)
    shapes = [((40, 64), torch.bfloat16), ((64,), torch.bfloat16), ((96, 32), torch.float32),
              ((32, 96), torch.bfloat16), ((128,), torch.float32), ((24, 40), torch.float16),
              ((300,), torch.bfloat16), ((72, 48), torch.bfloat16)]
    inits = [(torch.randn(s, generator=gen) * 0.02).to(dt) for s, dt in shapes]
    grads = [[(torch.randn(s, generator=gen) * 1e-3).to(dt) for s, dt in shapes] for _ in range(4)]

    def build(device):
        named = []
        for i, t in enumerate(inits):
            if i == 3 and device.type == "cpu":  # a transposed view of [96, 32] host storage
                p = nn.Parameter(t.t().contiguous().t())
                assert not p.is_contiguous()
            else:
                p = nn.Parameter(t.clone().to(device))
            named.append(("p%d" % i, p))
        return named, Gefen(named, lr=1e-3, weight_decay=0.01, fused=False, factored_v_2d=factored)

    runs = []
    for device in (dev, torch.device("cpu")):
        named, opt = build(device)
        for s, gs in enumerate(grads):
            for i, ((_, p), g) in enumerate(zip(named, gs)):
                p.grad = None if (s == 2 and i == 5) else g.clone().to(device)
            opt.step()
        torch.cuda.synchronize()
        runs.append((named, opt))
    (dn, dopt), (hn, hopt) = runs
    assert torch.equal(dopt._gefen_codebook.cpu(), hopt._gefen_codebook.cpu())
    for (n, pd), (_, ph) in zip(dn, hn):
        assert ph.device.type == "cpu"
        assert torch.equal(pd.detach().cpu(), ph.detach()), n
        for k, v in hopt.state[ph].items():
            if torch.is_tensor(v):
                assert v.device.type == "cpu", (n, k)
                assert torch.equal(dopt.state[pd][k].cpu(), v), (n, k)


def test_periodic_codebook_refresh_on_host(dev):
    """Reference tests/test_cpu_resident_step.py:75-101: codebook_refresh_every
    re-learns the codebook and remaps the stored indices with every
    parameter in host memory; the codebook and state stay on the host, and
    the run equals the same run on the GPU bit for bit."""
    from gefen import Gefen

    def run(device):
        torch.manual_seed(0)
        model = nn.Sequential(nn.Linear(32, 48), nn.Tanh(), nn.Linear(48, 16)).to(device)
        opt = Gefen(list(model.named_parameters()), lr=1e-3, fused=False, codebook_refresh_every=2)
        gen = torch.Generator().manual_seed(7)
        for _ in range(5):
            for p in model.parameters():
                p.grad = (torch.randn(p.shape, generator=gen) * 1e-2).to(device)
            opt.step()
            opt.zero_grad()
        return model, opt

    hm, ho = run(torch.device("cpu"))
    dm, do = run(dev)
    assert ho._gefen_codebook.device.type == "cpu"
    assert torch.equal(ho._gefen_codebook, do._gefen_codebook.cpu())
    for ph, pd in zip(hm.parameters(), dm.parameters()):
        assert torch.equal(ph.detach(), pd.detach().cpu())
        for k, v in ho.state[ph].items():
            if torch.is_tensor(v):
                assert v.device.type == "cpu", k
                assert torch.equal(v, do.state[pd][k].cpu()), k
