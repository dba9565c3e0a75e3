"""Capturable step: graph capture and replay of Gefen.step().

Contract of the reference's capturable mode (tests/test_capturable.py:1-31):
with capturable=True the step counters and the bias corrections derived from
them live on the device, a tensor lr is read on the device, and step() can be
captured into a CUDA/HIP graph after eager warm-up steps and replayed with
correct step-dependent math; with capturable=False capture raises.

Checks here:
  * eager parity: capturable=True steps like capturable=False (factored and
    block second moment, stochastic rounding on and off), counters are 0-dim
    fp32 device tensors;
  * lockstep replay: one optimizer replays a captured step while a twin steps
    eagerly with the same grads and tensor-lr schedule; after EVERY replay
    (with the twin's eager work in between) indices and magnitudes are
    bit-exact, second moments within 1e-6 and parameters within one bf16 ulp;
  * anti-freeze: after the last replay the scalar rows hold exactly the
    final step's [lr, 1/sqrt(bc2) or 1/bc2, 1/bc1, 1 - lr*wd] (the float64
    chain cast to fp32, gefen.py:1984-2001), none of the capture-time values;
  * the global step and rounding seed advance once per replay, also with no
    gradients; state_dict reports the replayed global step;
  * guards: capture with capturable=False, or before the first eager step;
  * checkpoints convert counters across the capturable toggle.
"""
import copy
import math

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GEFEN_SPECS = [("w2d", (48, 64)), ("norm", (64,)), ("bias", (48,))]
# Qwen-like mix: GQA projections, a transposed-view o_proj, an embedding, norms
# and a strided 1D view (stepped by the single-tensor path).
MIXED_SPECS = [("embed", (512, 64)), ("q_proj", (256, 64)), ("k_proj", (64, 64)), ("o_proj.t", (64, 256)),
               ("gate_proj", (192, 64)), ("down_proj.t", (64, 192)), ("input_norm", (64,)),
               ("q_norm", (32,)), ("strided", (96,))]
WD = 0.01
BETAS = (0.9, 0.999)


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _say(msg):
    print(msg, flush=True)


def _make_params(seed, specs, dtype, dev):
    gen = torch.Generator().manual_seed(seed)
    out = []
    for name, shape in specs:
        data = torch.randn(*shape, generator=gen) * 0.02
        if name.endswith(".t"):
            p = torch.nn.Parameter(data.t().contiguous().to(dtype).to(dev).t())
        elif name == "strided":
            base = torch.randn(2 * shape[0], generator=gen) * 0.02
            base[::2] = data
            p = torch.nn.Parameter(base.to(dtype).to(dev)[::2])
        else:
            p = torch.nn.Parameter(data.to(dtype).to(dev))
        out.append((name, p))
    return out


def _grads(seed, specs, steps, dtype, dev):
    gen = torch.Generator().manual_seed(seed)
    return [[(torch.randn(*shape, generator=gen) * 0.1).to(dtype).to(dev) for _, shape in specs]
            for _ in range(steps)]


def _make_opt(params, lr, factored, sr, capturable=True):
    from gefen import Gefen
    return Gefen(params, lr=lr, betas=BETAS, weight_decay=WD, factored_v_2d=factored, stochastic_round=sr,
                 capturable=capturable)


def _compare(opt_a, params_a, opt_b, params_b, tag):
    for (name, pa), (_, pb) in zip(params_a, params_b):
        sa, sb = opt_a.state[pa], opt_b.state[pb]
        for k in ("m_codebook", "m_magnitude"):
            if k in sa or k in sb:
                assert torch.equal(sa[k], sb[k]), "%s %s %s" % (tag, name, k)
        for k in ("v_row", "v_col", "vmean", "normuon_v", "exp_avg", "exp_avg_sq"):
            if k in sa:
                torch.testing.assert_close(sa[k], sb[k], rtol=1e-6, atol=0, msg="%s %s %s" % (tag, name, k))
        torch.testing.assert_close(pa.detach().float(), pb.detach().float(), rtol=2.0 ** -7, atol=1e-9,
                                   msg="%s %s param" % (tag, name))


def _counter_values(opt):
    out = set()
    for st in opt.state.values():
        for k in ("step", "vmean_step", "factored_step", "normuon_step"):
            if k in st:
                v = st[k]
                assert torch.is_tensor(v) and v.is_cuda and v.dim() == 0 and v.dtype == torch.float32, (k, v)
                out.add(v.item())
    return out


@pytest.mark.parametrize("factored", [True, False])
@pytest.mark.parametrize("sr", [False, True])
def test_eager_capturable_matches_host_scalars(dev, factored, sr):
    """Layer 1: capturable=True eager stepping equals capturable=False."""
    _say("eager parity factored=%s sr=%s" % (factored, sr))
    steps = 6
    dtype = torch.bfloat16 if sr else torch.float32  # rounding seeds matter for 16-bit parameters
    grads = _grads(1, GEFEN_SPECS, steps, dtype, dev)
    runs = []
    for capturable in (False, True):
        params = _make_params(0, GEFEN_SPECS, dtype, dev)
        opt = _make_opt(params, 1e-3, factored, sr, capturable)
        for i in range(steps):
            for (_, p), g in zip(params, grads[i]):
                p.grad = g.clone()
            opt.step()
        runs.append((opt, params))
    torch.cuda.synchronize()
    _compare(runs[1][0], runs[1][1], runs[0][0], runs[0][1], "capturable vs host")
    assert _counter_values(runs[1][0]) == {float(steps)}
    assert runs[1][0].state_dict()["gefen_global_step"] == steps


def _lockstep(dev, specs, dtype, factored, sr, warmup=3, replays=4, lr_start=1e-3, lr_decay=0.9, seed=0,
              make=None):
    """Captured optimizer vs eager twin, compared after every step."""
    steps = warmup + replays
    lr_sched = [lr_start * lr_decay ** i for i in range(steps)]
    grads = _grads(seed + 1, specs, steps, dtype, dev)
    make = make or (lambda ps, lr_: _make_opt(ps, lr_, factored, sr))
    ref_params = _make_params(seed, specs, dtype, dev)
    ref_lr = torch.tensor(lr_start, device=dev)
    ref_opt = make(ref_params, ref_lr)
    params = _make_params(seed, specs, dtype, dev)
    lr = torch.tensor(lr_start, device=dev)
    opt = make(params, lr)
    static = [torch.zeros_like(p) for _, p in params]
    for (_, p), sg in zip(params, static):
        p.grad = sg

    def ref_step(i):
        for (_, p), g in zip(ref_params, grads[i]):
            p.grad = g.clone()
        ref_lr.fill_(lr_sched[i])
        ref_opt.step()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for i in range(warmup):
            for sg, g in zip(static, grads[i]):
                sg.copy_(g)
            lr.fill_(lr_sched[i])
            opt.step()
    torch.cuda.current_stream().wait_stream(side)
    for i in range(warmup):
        ref_step(i)
    torch.cuda.synchronize()
    _compare(opt, params, ref_opt, ref_params, "warmup")

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt.step()
    for i in range(warmup, steps):
        for sg, g in zip(static, grads[i]):
            sg.copy_(g)
        lr.fill_(lr_sched[i])
        graph.replay()
        ref_step(i)  # eager work between replays
        torch.cuda.synchronize()
        _compare(opt, params, ref_opt, ref_params, "replay %d" % (i - warmup))
    return opt, params, ref_opt, steps, lr_sched, graph


@pytest.mark.parametrize("factored", [True, False])
@pytest.mark.parametrize("sr", [False, True])
def test_graph_replay_matches_eager_every_step(dev, factored, sr):
    dtype = torch.bfloat16 if sr else torch.float32
    _say("lockstep replay GEFEN_SPECS %s factored=%s sr=%s" % (dtype, factored, sr))
    opt, params, ref_opt, steps, lr_sched, _ = _lockstep(dev, GEFEN_SPECS, dtype, factored, sr)
    assert _counter_values(opt) == {float(steps)}
    # anti-freeze, exactly (the reference's legacy-vmean graph test,
    # tests/test_capturable.py:371-424)
    warmup = 3

    def f32(x):
        return float(np.float32(x))

    def expected(k, lr_value, factored_path):
        bc2 = 1.0 - BETAS[1] ** k
        lr32 = f32(lr_value)
        return [lr32, f32(1.0 / bc2) if factored_path else f32(1.0 / math.sqrt(bc2)),
                f32(1.0 / (1.0 - BETAS[0] ** k)), f32(1.0 - lr32 * WD)]

    for (name, p) in params:
        fact = factored and p.ndim == 2
        got = [float(x) for x in opt.state[p]["_capt_scalars"].cpu().tolist()]
        assert got == expected(steps, lr_sched[-1], fact), (name, got)
        frozen = expected(warmup + 1, lr_sched[warmup - 1], fact)
        assert all(g != f for g, f in zip(got, frozen)), (name, got, frozen)
    sd = opt.state_dict()
    assert sd["gefen_global_step"] == steps
    assert {int(c.item()) for c in opt._gefen_global_step_by_device.values()} == {steps}
    if sr:
        assert {int(s.item()) for s in opt._sr_seed_by_device.values()} == {steps}
    assert "_capt_scalars" not in next(iter(sd["state"].values()))


@pytest.mark.parametrize("factored", [True, False])
def test_graph_replay_mixed_set_bf16(dev, factored):
    """Several kernel variants in one plan (contiguous, transposed views, 1D)
    plus a strided parameter stepped by the single-tensor path inside the
    captured step."""
    _say("lockstep replay MIXED_SPECS bf16 factored=%s" % factored)
    opt, params, _, steps, _, _ = _lockstep(dev, MIXED_SPECS, torch.bfloat16, factored, False, warmup=2,
                                            replays=5, seed=7)
    assert not dict(params)["o_proj.t"].is_contiguous()
    assert _counter_values(opt) == {float(steps)}


def test_schedule_is_not_baked(dev):
    """A constant-lr captured run lands elsewhere than a scheduled one."""
    _say("schedule bites")
    a = _lockstep(dev, GEFEN_SPECS, torch.float32, True, False, lr_decay=0.5)
    b = _lockstep(dev, GEFEN_SPECS, torch.float32, True, False, lr_decay=1.0)
    diff = max((pa.detach() - pb.detach()).abs().max().item() for (_, pa), (_, pb) in zip(a[1], b[1]))
    assert diff > 5e-5, diff


def test_global_step_advances_without_gradients(dev):
    """tests/test_capturable.py:774-790: replays advance the global step
    even when no parameter has a gradient."""
    _say("global step without grads")
    from gefen import Gefen
    p = torch.nn.Parameter(torch.ones(32, device=dev))
    opt = Gefen([("unused", p)], lr=1e-3, capturable=True)
    for _ in range(2):
        opt.step()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt.step()
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    assert opt.state_dict()["gefen_global_step"] == 5


def test_capture_without_capturable_raises(dev):
    _say("guard: capturable=False")
    from gefen import Gefen
    params = _make_params(0, GEFEN_SPECS, torch.float32, dev)
    opt = Gefen(params, lr=1e-3)
    for (_, p), g in zip(params, _grads(1, GEFEN_SPECS, 1, torch.float32, dev)[0]):
        p.grad = g
    opt.step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="capturable=False"):
        with torch.cuda.graph(graph):
            opt.step()


def test_capture_before_first_step_raises(dev):
    _say("guard: capture before step 1")
    params = _make_params(0, GEFEN_SPECS, torch.float32, dev)
    opt = _make_opt(params, 1e-3, True, False)
    for (_, p), g in zip(params, _grads(1, GEFEN_SPECS, 1, torch.float32, dev)[0]):
        p.grad = g
    graph = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="eager step"):
        with torch.cuda.graph(graph):
            opt.step()


def test_state_dict_roundtrip_across_toggle(dev):
    """tests/test_capturable.py:635-686: counters become python ints in a
    plain optimizer and 0-dim fp32 device tensors in a capturable one; both
    keep stepping."""
    _say("checkpoint across the capturable toggle")
    steps = 3
    grads = _grads(2, GEFEN_SPECS, steps + 1, torch.float32, dev)

    def run(capturable):
        params = _make_params(0, GEFEN_SPECS, torch.float32, dev)
        opt = _make_opt(params, 1e-3, True, False, capturable)
        for i in range(steps):
            for (_, p), g in zip(params, grads[i]):
                p.grad = g.clone()
            opt.step()
        return params, opt

    _, cap = run(True)
    params_plain = _make_params(0, GEFEN_SPECS, torch.float32, dev)
    plain = _make_opt(params_plain, 1e-3, True, False, False)
    plain.load_state_dict(cap.state_dict())
    for st in plain.state.values():
        for k in ("step", "factored_step", "vmean_step"):
            if k in st:
                assert isinstance(st[k], int) and st[k] == steps, (k, st[k])
    for (_, p), g in zip(params_plain, grads[steps]):
        p.grad = g.clone()
    plain.step()

    p2, plain2 = run(False)
    params_cap = [(name, torch.nn.Parameter(p.detach().clone())) for name, p in p2]
    cap2 = _make_opt(params_cap, 1e-3, True, False, True)
    cap2.load_state_dict(copy.deepcopy(plain2.state_dict()))  # loading shares same-device state tensors
    assert _counter_values(cap2) == {float(steps)}
    assert cap2._gefen_global_step == steps
    for (_, p), g in zip(params_cap, grads[steps]):
        p.grad = g.clone()
    cap2.step()
    for (_, p), g in zip(p2, grads[steps]):
        p.grad = g.clone()
    plain2.step()
    torch.cuda.synchronize()
    _compare(cap2, params_cap, plain2, p2, "capturable resumed vs plain")
    assert _counter_values(cap2) == {float(steps + 1)}


def test_capture_with_grads_produced_in_graph(dev):
    """Whole-step capture: the grads are produced inside the captured region
    (new tensors from the graph's pool, as a captured backward makes them), so
    the launch plan is built during the capture and its descriptor upload is
    part of every replay."""
    _say("grads produced inside the capture")
    steps, warmup = 6, 2
    specs = MIXED_SPECS[:4] + MIXED_SPECS[6:8]
    grads = _grads(5, specs, steps, torch.bfloat16, dev)
    ref_params = _make_params(4, specs, torch.bfloat16, dev)
    ref_opt = _make_opt(ref_params, 1e-3, True, False)
    params = _make_params(4, specs, torch.bfloat16, dev)
    opt = _make_opt(params, 1e-3, True, False)
    src = [torch.zeros_like(g) for g in grads[0]]

    def produce_grads():
        for (_, p), s in zip(params, src):
            p.grad = s * 1.0

    for i in range(steps):
        for s, g in zip(src, grads[i]):
            s.copy_(g)
        for (_, p), g in zip(ref_params, grads[i]):
            p.grad = g.clone()
        ref_opt.step()
        if i < warmup:
            produce_grads()
            opt.step()
            continue
        if i == warmup:
            for _, p in params:
                p.grad = None
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                produce_grads()
                opt.step()
        graph.replay()
        torch.cuda.synchronize()
        _compare(opt, params, ref_opt, ref_params, "in-graph grads step %d" % i)
    assert opt.state_dict()["gefen_global_step"] == steps


MUON_SPECS = [("h1", (64, 48)), ("h2", (32, 64)), ("h3", (64, 48))]
HYBRID_MUON_SPECS = [("h1.weight", (64, 48)), ("h2.weight", (32, 64))]
HYBRID_BACKUP_SPECS = [("embed.weight", (96, 32)), ("norm.weight", (64,))]


def _muon(params, lr, sr=False, capturable=True, cautious=False):
    from gefen import GefenMuon
    return GefenMuon(params, lr=lr, weight_decay=WD, normuon=True, stochastic_round=sr, capturable=capturable,
                     cautious=cautious)


def _hybrid(params, lr, backup="gefen", sr=False, capturable=True):
    from gefen import GefenMuonHybrid
    n = len(HYBRID_MUON_SPECS)
    return GefenMuonHybrid(params[:n], params[n:], lr=lr, backup_optimizer=backup, weight_decay=WD,
                           stochastic_round=sr, capturable=capturable)


@pytest.mark.parametrize("sr", [False, True])
def test_muon_eager_capturable_matches_host_scalars(dev, sr):
    """GefenMuon (NorMuon on): capturable eager stepping equals the host path;
    step and normuon_step are device counters."""
    _say("muon eager parity sr=%s" % sr)
    steps, dtype = 5, torch.bfloat16
    grads = _grads(3, MUON_SPECS, steps, dtype, dev)
    runs = []
    for capturable in (False, True):
        params = _make_params(2, MUON_SPECS, dtype, dev)
        opt = _muon(params, 1e-3, sr, capturable)
        for i in range(steps):
            for (_, p), g in zip(params, grads[i]):
                p.grad = g.clone()
            opt.step()
        runs.append((opt, params))
    torch.cuda.synchronize()
    _compare(runs[1][0], runs[1][1], runs[0][0], runs[0][1], "muon capturable vs host")
    assert _counter_values(runs[1][0]) == {float(steps)}
    assert any("normuon_step" in st for st in runs[1][0].state.values())


@pytest.mark.parametrize("sr", [False, True])
def test_muon_graph_replay_matches_eager_every_step(dev, sr):
    _say("muon lockstep replay sr=%s" % sr)
    opt, params, _, steps, lr_sched, _ = _lockstep(dev, MUON_SPECS, torch.bfloat16, False, sr, seed=11,
                                                   make=lambda ps, lr: _muon(ps, lr, sr))
    assert _counter_values(opt) == {float(steps)}
    for _, p in params:
        got = [float(x) for x in opt.state[p]["_capt_scalars"].cpu().tolist()]
        lr32 = float(np.float32(lr_sched[-1]))
        assert got[0] == lr32 and got[3] == float(np.float32(1.0 - lr32 * WD)), got
    assert opt.state_dict()["gefen_global_step"] == steps


def test_muon_cautious_graph_replay_matches_eager_every_step(dev):
    """Cautious masking inside a captured step: its counters are cleared by a
    kernel, so every replay recounts."""
    _say("muon cautious lockstep replay")
    opt, params, _, steps, _, _ = _lockstep(dev, MUON_SPECS, torch.bfloat16, False, False, seed=13,
                                            make=lambda ps, lr: _muon(ps, lr, cautious=True))
    assert _counter_values(opt) == {float(steps)}


@pytest.mark.parametrize("backup", ["gefen", "adamw"])
def test_hybrid_graph_replay_matches_eager_every_step(dev, backup):
    _say("hybrid lockstep replay backup=%s" % backup)
    specs = HYBRID_MUON_SPECS + HYBRID_BACKUP_SPECS
    opt, params, _, steps, _, _ = _lockstep(dev, specs, torch.float32, False, False, seed=21,
                                            make=lambda ps, lr: _hybrid(ps, lr, backup))
    assert _counter_values(opt.muon) == {float(steps)}
    if backup == "gefen":
        assert _counter_values(opt.backup) == {float(steps)}


@pytest.mark.parametrize("factored", [True, False])
@pytest.mark.parametrize("sr", [False, True])
def test_graph_replay_matches_oracle(dev, factored, sr):
    """Captured-and-replayed steps against the oracle directly (not only
    against eager HIP): 3 eager steps (step 1 learns the period and the
    codebook), then 4 replays of one captured step with fresh grads copied
    into the static grad buffers and a device lr schedule.  After every step,
    each parameter's indices and magnitudes are bit-exact with the oracle's
    step (stochastic rounding seeded with the global step, as the reference's
    device seed is), second moments within 1e-6 and parameters within one
    bf16 ulp.  The oracle continues from the GPU's parameters and second
    moments each step, so summation-order skew does not accumulate."""
    from oracle import oracle as orc
    from local_checks import assert_within_ulp
    _say("replay vs oracle factored=%s sr=%s" % (factored, sr))
    specs = [("w2d", (48, 64)), ("norm", (64,)), ("w2d_b", (32, 96))]
    dtype = torch.bfloat16
    warmup, replays = 3, 4
    steps = warmup + replays
    lr_sched = [1e-3 * 0.9 ** i for i in range(steps)]
    grads = _grads(11, specs, steps, dtype, dev)
    params = _make_params(5, specs, dtype, dev)
    lr = torch.tensor(lr_sched[0], device=dev)
    opt = _make_opt(params, lr, factored, sr)
    static = [torch.zeros_like(p) for _, p in params]
    for (_, p), sg in zip(params, static):
        p.grad = sg
    ref = {name: {"p": p.detach().float().cpu().numpy()} for name, p in params}
    graph = None
    side = torch.cuda.Stream()
    for i in range(steps):
        for sg, g in zip(static, grads[i]):
            sg.copy_(g)
        lr.fill_(lr_sched[i])
        if i < warmup:
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                opt.step()
            torch.cuda.current_stream().wait_stream(side)
        else:
            if graph is None:
                torch.cuda.synchronize()
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph):
                    opt.step()
            graph.replay()
        torch.cuda.synchronize()
        s = i + 1
        cb = opt._gefen_codebook.cpu().numpy()
        lr32 = float(np.float32(lr_sched[i]))
        kw = dict(beta1=BETAS[0], beta2=BETAS[1], lr=lr32, eps=1e-8, bc1=1 - BETAS[0] ** s,
                  bc2=1 - BETAS[1] ** s, wd=WD, sr_seed=(i if sr else None))
        for (name, p), g in zip(params, grads[i]):
            st = opt.state[p]
            r = ref[name]
            per = int(st["automatic_period"])
            gn = g.float().cpu().numpy()
            if "idx" not in r:
                r["idx"] = np.zeros(p.numel(), np.uint8)
                r["mag"] = np.zeros(p.numel() // per, np.float32)
                r["v_row"] = np.zeros(p.shape[0], np.float32)
                r["v_col"] = np.zeros(p.shape[-1], np.float32)
                r["vmean"] = np.zeros(p.numel() // per, np.float32)
            if factored and p.ndim == 2:
                pn, r["idx"], r["mag"], vr, vc = orc.factored_step(
                    r["p"], gn, r["idx"], r["mag"], r["v_row"], r["v_col"], per, cb, orc.BF16, **kw)
                np.testing.assert_allclose(st["v_row"].cpu().numpy(), vr, rtol=1e-6)
                np.testing.assert_allclose(st["v_col"].cpu().numpy(), vc, rtol=1e-6)
                r["v_row"], r["v_col"] = st["v_row"].cpu().numpy(), st["v_col"].cpu().numpy()
            else:
                pn, r["idx"], r["mag"], vm = orc.block_step(
                    r["p"], gn, r["idx"], r["mag"], r["vmean"], per, cb, orc.BF16, **kw)
                np.testing.assert_allclose(st["vmean"].cpu().numpy().reshape(-1), vm, rtol=1e-6)
                r["vmean"] = st["vmean"].cpu().numpy().reshape(-1)
            tag = "%s step %d (%s)" % (name, s, "eager" if i < warmup else "replay")
            np.testing.assert_array_equal(st["m_codebook"].cpu().numpy().reshape(-1), r["idx"], err_msg=tag)
            np.testing.assert_array_equal(st["m_magnitude"].cpu().numpy().reshape(-1), r["mag"], err_msg=tag)
            got = p.detach().float().cpu().numpy()
            assert_within_ulp(got, pn, orc.BF16, tag + " p", atol=1e-6 * lr32)
            r["p"] = got
    assert opt.state_dict()["gefen_global_step"] == steps
