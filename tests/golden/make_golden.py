"""Generate golden input/output vectors from the reference's CPU step.

Runs ONLY in the build container, where the reference checkout is mounted
read-only at /root/reference.  It imports the reference package ``gefen`` from
/root/reference/src and records small seeded fixtures (inputs and the
reference's outputs) as .npz files next to this script.  Nothing at test time
reads the reference: the tests load the committed .npz fixtures.

Cases (each a separate file so they can be regenerated independently):
  nearest.npz      gefen_nearest_codebook_indices        gefen.py:288-334
  lut.npz          _codebook_search_lut                 kernels/automatic_gefen_fused.py:81-121
  dp.npz           quantization.exact_dp (pure-Python)  quantization.py:197-253
  learn.npz        learn_gefen_exact_codebook_from_grad_periods gefen.py:417-517
  period.npz       find_period_by_block_variance (cpu)  partitioning.py:274-313
  step_<name>.npz  Gefen(fused=False).step trajectories  gefen.py:2784-3018, 3488-3818
  config1.npz      config-1 trajectory (4096x4096 fp32 + 4096 bias, 10 steps);
                   large arrays are stored as sha256 digests plus subsamples.
  muon_ns.npz      _zeropower_via_newtonschulz on bf16 inputs gefen_muon.py:236-291
  muon_<dt>.npz    GefenMuon(fused=False) trajectories         gefen_muon.py:2945-3030
  hybrid_bf16.npz  GefenMuonHybrid(fused=False) trajectory      hybrid.py:693-776
  ckpt_<name>.pt   a reference-written Gefen checkpoint            gefen.py:4558-4707
  ckpt_<name>.npz  the reference's trajectory after loading it     gefen.py:5456-5707

Usage:  python tests/golden/make_golden.py [case ...]   (default: all but config1)
"""
from __future__ import annotations

import hashlib
import os
import sys
import time
import warnings

import numpy as np
import torch

REF_SRC = "/root/reference/src"
HERE = os.path.dirname(os.path.abspath(__file__))

# Hyperparameters of BASELINE config 1 (shared by every trajectory case).
LR, BETAS, EPS, WD = 6e-5, (0.9, 0.999), 1e-8, 0.01


def _ref():
    if REF_SRC not in sys.path:
        sys.path.insert(0, REF_SRC)
    import gefen  # noqa: F401  (the reference package)
    return gefen


def _save(name, **arrays):
    path = os.path.join(HERE, name)
    np.savez_compressed(path, **arrays)
    print("wrote", path, sorted(arrays), flush=True)


def _f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float32).cpu().numpy().copy()


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


# ----------------------------------------------------------------- search


def _test_codebook(seed=7, k=256, dup=True):
    g = torch.Generator().manual_seed(seed)
    inner = torch.sort(torch.rand(k - 2, generator=g) * 2 - 1).values
    cb = torch.cat([torch.tensor([-1.0]), inner, torch.tensor([1.0])]).float()
    if dup and k >= 8:
        cb[k // 2] = cb[k // 2 - 1]  # a duplicated codeword
    return torch.sort(cb).values


def _probe_values(cb: torch.Tensor, seed=11, n=4000):
    g = torch.Generator().manual_seed(seed)
    vals = [torch.rand(n, generator=g) * 2.2 - 1.1, cb.clone()]
    mids = (cb[:-1] + cb[1:]) / 2
    vals += [mids, torch.nextafter(mids, torch.full_like(mids, 2.0)),
             torch.nextafter(mids, torch.full_like(mids, -2.0))]
    vals.append(torch.tensor([0.0, -0.0, 1.0, -1.0, 1.5, -1.5,
                              float("inf"), float("-inf")]))
    return torch.cat(vals).float()


def case_nearest():
    ref = _ref()
    from gefen.gefen import gefen_nearest_codebook_indices as near
    out = {}
    for tag, cb in (("k256", _test_codebook()), ("k1", torch.tensor([0.25])),
                    ("k2", torch.tensor([-1.0, 1.0])),
                    ("k3", torch.tensor([-1.0, 0.0, 1.0]))):
        x = _probe_values(cb)
        out["cb_" + tag] = _f32(cb)
        out["x_" + tag] = _f32(x)
        out["idx_" + tag] = near(cb, x).numpy().copy()
    del ref
    _save("nearest.npz", **out)


def case_lut():
    _ref()
    from gefen.kernels.automatic_gefen_fused import _codebook_search_lut
    out = {}
    for tag, cb in (("rand", _test_codebook()),
                    ("dense", torch.linspace(-1, 1, 256)),
                    ("k3", torch.tensor([-1.0, 0.0, 1.0]))):
        out["cb_" + tag] = _f32(cb)
        out["lut_" + tag] = _codebook_search_lut(cb.float()).numpy().copy()
    _save("lut.npz", **out)


# ----------------------------------------------------------------- exact DP


def _hist_stats(counts: torch.Tensor):
    bins = counts.numel()
    edges = torch.linspace(-1.0, 1.0, steps=bins + 1, dtype=torch.float32)
    centers = 0.5 * (edges[:-1] + edges[1:])
    c = counts.to(torch.float32)
    act = c > 0
    return {"bin_edges": edges, "bin_centers": centers, "bin_counts": c,
            "active_bins": act, "active_centers": centers[act],
            "active_counts": c[act], "active_sums": centers[act] * c[act]}


def _synthetic_counts(seed, n_active, bins=4096):
    g = torch.Generator().manual_seed(seed)
    counts = torch.zeros(bins, dtype=torch.int64)
    pos = torch.randperm(bins, generator=g)[:n_active]
    counts[pos] = torch.randint(1, 5000, (n_active,), generator=g)
    return counts


def case_dp():
    _ref()
    import gefen.quantization as q
    out = {}
    for tag, seed, n_act in (("pad40", 1, 40), ("a300", 2, 300), ("a520", 3, 520)):
        counts = _synthetic_counts(seed, n_act)
        t0 = time.time()
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            cb = q.exact_dp(histogram_stats=_hist_stats(counts), num_codebooks=256,
                            force_endpoints=True)
        print("  dp", tag, "%.1fs" % (time.time() - t0), flush=True)
        out["counts_" + tag] = counts.numpy().copy()
        out["cb_" + tag] = _f32(cb)
    _save("dp.npz", **out)


def _learn_inputs():
    g = torch.Generator().manual_seed(21)
    w = torch.randn(16, 24, generator=g) * 1e-3
    b = torch.randn(40, generator=g) * 1e-3
    return [("w", w, 24), ("b", b, 8)]


def case_learn():
    _ref()
    from gefen.gefen import learn_gefen_exact_codebook_from_grad_periods as learn
    items = _learn_inputs()
    gp = [(n, t.reshape(-1), p, t) for n, t, p in items]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        cb = learn(grad_periods=iter(gp), codebook_device=torch.device("cpu"),
                   num_codebooks=256, force_endpoints=True, verbose=False,
                   compute_mse_logging=False, use_fused_histogram=False)
    out = {"cb": _f32(cb)}
    for n, t, p in items:
        out["g_" + n] = _f32(t)
        out["period_" + n] = np.int64(p)
    _save("learn.npz", **out)


# ------------------------------------------------------------ period search


PERIOD_SHAPES = {"m64x96": (64, 96), "v4096": (4096,), "t105": (3, 5, 7),
                 "v1000": (1000,), "v128": (128,), "m24x24": (24, 24),
                 "m12x4096": (12, 4096)}


def case_period():
    _ref()
    from gefen.partitioning import find_period_by_block_variance, divisors
    from gefen.partitioning import average_within_block_variance_cpu
    out = {}
    for i, (tag, shape) in enumerate(PERIOD_SHAPES.items()):
        gen = torch.Generator().manual_seed(300 + i)
        g = torch.randn(*shape, generator=gen) * 1e-3
        if tag == "m12x4096":  # row-structured scale so a real period exists
            g = g * (torch.arange(12, dtype=torch.float32) + 1.0).view(12, 1) ** 2
        vals = g.float().square().reshape(-1).numpy()
        period = find_period_by_block_variance(vals, print_results=False,
                                               parameter_shape=tuple(shape),
                                               backend="cpu")
        errs = [average_within_block_variance_cpu(vals, d) for d in divisors(vals.size)]
        out["g_" + tag] = _f32(g)
        out["period_" + tag] = np.int64(period)
        out["errs_" + tag] = np.array(errs, dtype=np.float64)
    _save("period.npz", **out)


# --------------------------------------------------------------- trajectories


def _golden_codebook() -> torch.Tensor:
    path = os.path.join(HERE, "learn.npz")
    if not os.path.exists(path):
        case_learn()
    return torch.from_numpy(np.load(path)["cb"]).float()


STEP_CASES = {
    # name: (dtype, factored, [(pname, shape, period or None)], wd, steps)
    "fact_f32": (torch.float32, True, [("w", (48, 80), None), ("b", (80,), None)], WD, 10),
    "fact_bf16": (torch.bfloat16, True, [("w", (40, 64), 16), ("b", (64,), 8)], WD, 6),
    "fact_f16": (torch.float16, True, [("w", (24, 40), 40), ("b", (40,), 40)], 0.0, 4),
    "block_bf16": (torch.bfloat16, False, [("w", (32, 48), 48), ("b", (48,), 1)], WD, 6),
    "block_f32": (torch.float32, False, [("w", (16, 30), 480), ("b", (30,), 30)], 0.0, 5),
    "block_f16": (torch.float16, False, [("w", (16, 32), 64), ("b", (32,), 8)], WD, 4),
    "zeros_f32": (torch.float32, False, [("w", (8, 16), 16)], WD, 3),
}


def step_case_inputs(name):
    """Seeded params/grads of a trajectory case (shared with the tests)."""
    dtype, factored, specs, wd, steps = STEP_CASES[name]
    gen = torch.Generator().manual_seed(0)
    params = [(pn, (torch.randn(*shape, generator=gen) * 0.02).to(dtype), per)
              for pn, shape, per in specs]
    grads = []
    for t in range(1, steps + 1):
        gt = torch.Generator().manual_seed(1000 + t)
        step_grads = []
        for pn, shape, _ in specs:
            gv = (torch.randn(*shape, generator=gt) * 1e-3).to(dtype)
            if name == "zeros_f32" and t == 1:
                gv.view(-1)[:16] = 0  # block 0 stays all-zero: magnitude 0 path
            step_grads.append(gv)
        grads.append(step_grads)
    return dtype, factored, params, grads, wd, steps


def run_reference_trajectory(params, grads, *, factored, wd, codebook,
                             periods=None, record=None):
    ref = _ref()
    from gefen import Gefen
    ps = [(n, torch.nn.Parameter(t.clone())) for n, t, _ in params]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        opt = Gefen(ps, lr=LR, betas=BETAS, eps=EPS, weight_decay=wd,
                    fused=False, factored_v_2d=factored)
    if codebook is not None:
        opt._gefen_codebook = codebook.clone()
    for (n, t, per), (_, p) in zip(params, ps):
        if per is not None:
            opt.state[p]["automatic_period"] = int(per)
    traj = []
    for step_grads in grads:
        for (_, p), gv in zip(ps, step_grads):
            p.grad = gv.clone()
        opt.step()
        rec = {}
        for n, p in ps:
            st = opt.state[p]
            rec[n] = {"p": p.detach().clone(), "idx": st["m_codebook"].clone(),
                      "mag": st["m_magnitude"].clone(),
                      "period": int(st["automatic_period"])}
            for key in ("v_row", "v_col", "vmean"):
                if key in st:
                    rec[n][key] = st[key].clone()
        traj.append(rec if record is None else record(rec))
    del ref
    return opt, traj


def case_step(name):
    dtype, factored, params, grads, wd, steps = step_case_inputs(name)
    cb = _golden_codebook()
    opt, traj = run_reference_trajectory(params, grads, factored=factored, wd=wd,
                                         codebook=cb)
    out = {"codebook": _f32(cb), "wd": np.float64(wd), "steps": np.int64(steps),
           "factored": np.int64(factored)}
    for n, t, _ in params:
        out["p0_" + n] = _f32(t)
    for s, (step_grads, rec) in enumerate(zip(grads, traj), start=1):
        for (n, _, _), gv in zip(params, step_grads):
            out["g%d_%s" % (s, n)] = _f32(gv)
            r = rec[n]
            out["period_" + n] = np.int64(r["period"])
            out["p%d_%s" % (s, n)] = _f32(r["p"])
            out["idx%d_%s" % (s, n)] = r["idx"].numpy().reshape(-1).copy()
            out["mag%d_%s" % (s, n)] = _f32(r["mag"]).reshape(-1)
            for key in ("v_row", "v_col", "vmean"):
                if key in r:
                    out["%s%d_%s" % (key, s, n)] = _f32(r[key]).reshape(-1)
    _save("step_%s.npz" % name, **out)


# ------------------------------------------------------------------ config 1


def config1_inputs(step: int | None = None):
    """W 4096x4096 + b 4096 fp32 ~ N(0, 0.02) from seed 0;
    step-t grads ~ N(0, 1e-3) from seed 1000+t (W first, then b)."""
    gen = torch.Generator().manual_seed(0)
    w = torch.randn(4096, 4096, generator=gen) * 0.02
    b = torch.randn(4096, generator=gen) * 0.02
    if step is None:
        return w, b
    gt = torch.Generator().manual_seed(1000 + step)
    return torch.randn(4096, 4096, generator=gt) * 1e-3, torch.randn(4096, generator=gt) * 1e-3


SUB = 4099  # subsample stride for the 16.7M-element weight


def case_config1():
    ref = _ref()
    from gefen import Gefen
    w0, b0 = config1_inputs()
    W = torch.nn.Parameter(w0.clone())
    B = torch.nn.Parameter(b0.clone())
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        opt = Gefen([("weight", W), ("bias", B)], lr=LR, betas=BETAS, eps=EPS,
                    weight_decay=WD, fused=False, factored_v_2d=True)
    out = {}
    for s in range(1, 11):
        gw, gb = config1_inputs(s)
        W.grad, B.grad = gw, gb
        t0 = time.time()
        opt.step()
        print("  config1 step", s, "%.1fs" % (time.time() - t0), flush=True)
        sw, sb = opt.state[W], opt.state[B]
        if s == 1:
            out["codebook"] = _f32(opt._gefen_codebook)
            out["period_weight"] = np.int64(sw["automatic_period"])
            out["period_bias"] = np.int64(sb["automatic_period"])
        out["sha_idx%d_weight" % s] = np.array(sha(sw["m_codebook"].numpy()))
        out["idx_sub%d_weight" % s] = sw["m_codebook"].reshape(-1)[::SUB].numpy().copy()
        out["sha_p%d_weight" % s] = np.array(sha(W.detach().numpy()))
        out["p_sub%d_weight" % s] = W.detach().reshape(-1)[::SUB].numpy().copy()
        out["mag%d_weight" % s] = _f32(sw["m_magnitude"]).reshape(-1)
        out["v_row%d_weight" % s] = _f32(sw["v_row"])
        out["v_col%d_weight" % s] = _f32(sw["v_col"])
        out["p%d_bias" % s] = _f32(B)
        out["idx%d_bias" % s] = sb["m_codebook"].reshape(-1).numpy().copy()
        out["mag%d_bias" % s] = _f32(sb["m_magnitude"]).reshape(-1)
        out["vmean%d_bias" % s] = _f32(sb["vmean"]).reshape(-1)
        _save("config1.npz", **out)  # checkpoint after every step
    del ref


# ------------------------------------------------------------------- Muon

NS_CASES = {
    # name: (shape, schedule)  schedule None = standard (a, b, c) x 5
    "wide": ((48, 96), None),
    "tall": ((96, 40), None),
    "square": ((64, 64), "tuned3"),
    "wide4": ((32, 80), "tuned4"),
}


def case_muon_ns():
    """_zeropower_via_newtonschulz (gefen_muon.py:236-291) on bf16 inputs."""
    _ref()
    from gefen import gefen_muon as gm
    out = {}
    gen = torch.Generator().manual_seed(5)
    for name, (shape, sched) in NS_CASES.items():
        m = (torch.randn(*shape, generator=gen) * 1e-3).to(torch.bfloat16)
        coeffs = (gm.DEFAULT_A, gm.DEFAULT_B, gm.DEFAULT_C) if sched is None else gm.NS_SCHEDULES[sched]
        o = gm._zeropower_via_newtonschulz(m, coeffs, gm.DEFAULT_NS_STEPS, gm.EPS)
        out["in_" + name] = _f32(m)
        out["out_" + name] = _f32(o)
        sch = gm._normalize_ns_schedule(coeffs, gm.DEFAULT_NS_STEPS)
        out["abc_" + name] = np.array(sch, dtype=np.float64)
    # zero input: the eps clamp keeps the output zero
    z = torch.zeros(16, 24, dtype=torch.bfloat16)
    out["in_zero"] = _f32(z)
    out["out_zero"] = _f32(gm._zeropower_via_newtonschulz(
        z, (gm.DEFAULT_A, gm.DEFAULT_B, gm.DEFAULT_C), gm.DEFAULT_NS_STEPS, gm.EPS))
    _save("muon_ns.npz", **out)


MUON_CASES = {
    # name: (dtype, [(pname, shape, period)], kwargs, steps)
    "muon_bf16": (torch.bfloat16, [("a", (48, 80), 80), ("b", (80, 48), 16)],
                  dict(lr=0.02, weight_decay=0.1, momentum=0.95, nesterov=True), 4),
    "muon_f32": (torch.float32, [("a", (40, 64), 64), ("b", (64, 40), 40)],
                 dict(lr=0.02, weight_decay=0.1, momentum=0.9, nesterov=False,
                      adjust_lr_fn="match_rms_adamw", normuon=True), 3),
}


def muon_case_inputs(name):
    dtype, specs, kw, steps = MUON_CASES[name]
    gen = torch.Generator().manual_seed(3)
    params = [(pn, (torch.randn(*shape, generator=gen) * 0.02).to(dtype), per) for pn, shape, per in specs]
    grads = []
    for t in range(1, steps + 1):
        gt = torch.Generator().manual_seed(2000 + t)
        grads.append([(torch.randn(*shape, generator=gt) * 1e-3).to(dtype) for _, shape, _ in specs])
    return dtype, params, grads, kw, steps


def case_muon(name):
    """GefenMuon(fused=False) trajectory on the CPU (gefen_muon.py:2945-3030)."""
    _ref()
    from gefen import GefenMuon
    dtype, params, grads, kw, steps = muon_case_inputs(name)
    cb = _golden_codebook()
    ps = [(n, torch.nn.Parameter(t.clone())) for n, t, _ in params]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        opt = GefenMuon(ps, fused=False, **kw)
    opt._gefen_codebook = cb.clone()
    for (n, t, per), (_, p) in zip(params, ps):
        opt.state[p]["automatic_period"] = int(per)
    out = {"codebook": _f32(cb)}
    for n, t, per in params:
        out["p0_" + n] = _f32(t)
        out["period_" + n] = np.int64(per)
    for s_, step_grads in enumerate(grads, start=1):
        for (_, p), gv in zip(ps, step_grads):
            p.grad = gv.clone()
        opt.step()
        for (n, p), gv in zip(ps, step_grads):
            st = opt.state[p]
            out["g%d_%s" % (s_, n)] = _f32(gv)
            out["p%d_%s" % (s_, n)] = _f32(p.detach())
            out["idx%d_%s" % (s_, n)] = st["m_codebook"].reshape(-1).numpy().copy()
            out["mag%d_%s" % (s_, n)] = _f32(st["m_magnitude"]).reshape(-1)
            if "normuon_v" in st:
                out["nv%d_%s" % (s_, n)] = _f32(st["normuon_v"]).reshape(-1)
    _save("%s.npz" % name, **out)


def case_hybrid():
    """GefenMuonHybrid(fused=False) with its defaults (hybrid.py:228-265):
    two hidden matrices go to GefenMuon, an embedding and a norm vector to the
    block-vmean Gefen backup."""
    _ref()
    from gefen import GefenMuonHybrid
    gen = torch.Generator().manual_seed(4)
    specs = [("layers.0.mlp.w", (40, 72), 72, True), ("layers.0.attn.o", (72, 40), 24, True),
             ("embed_tokens.weight", (50, 16), 16, False), ("layers.0.norm.weight", (72,), 8, False)]
    dtype = torch.bfloat16
    tensors = {n: (torch.randn(*sh, generator=gen) * 0.02).to(dtype) for n, sh, _, _ in specs}
    muon = [(n, torch.nn.Parameter(tensors[n].clone())) for n, _, _, m in specs if m]
    backup = [(n, torch.nn.Parameter(tensors[n].clone())) for n, _, _, m in specs if not m]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        opt = GefenMuonHybrid(muon, backup, lr=1e-3, weight_decay=0.01, fused=False)
    cb = _golden_codebook()
    opt.muon._gefen_codebook = cb.clone()
    opt.backup._gefen_codebook = cb.clone()
    named = dict(muon + backup)
    for n, _, per, m in specs:
        (opt.muon if m else opt.backup).state[named[n]]["automatic_period"] = int(per)
    out = {"codebook": _f32(cb)}
    for n, sh, per, m in specs:
        out["p0_" + n] = _f32(tensors[n])
        out["period_" + n] = np.int64(per)
    for s_ in range(1, 4):
        gt = torch.Generator().manual_seed(3000 + s_)
        for n, sh, _, _ in specs:
            gv = (torch.randn(*sh, generator=gt) * 1e-3).to(dtype)
            named[n].grad = gv
            out["g%d_%s" % (s_, n)] = _f32(gv)
        opt.step()
        for n, sh, per, m in specs:
            st = (opt.muon if m else opt.backup).state[named[n]]
            out["p%d_%s" % (s_, n)] = _f32(named[n].detach())
            out["idx%d_%s" % (s_, n)] = st["m_codebook"].reshape(-1).numpy().copy()
            out["mag%d_%s" % (s_, n)] = _f32(st["m_magnitude"]).reshape(-1)
            for key in ("vmean", "normuon_v"):
                if key in st:
                    out["%s%d_%s" % (key, s_, n)] = _f32(st[key]).reshape(-1)
    _save("hybrid_bf16.npz", **out)


# --------------------------------------------------------------- checkpoints

CKPT_CASES = {
    # name: (trajectory case whose params/grads are used, steps before the checkpoint)
    "fact_bf16": ("fact_bf16", 3),
    "block_bf16": ("block_bf16", 3),
}


def case_checkpoint(name):
    """A reference-written checkpoint (ckpt_<name>.pt: Gefen.state_dict() after
    `pre` steps, period search and codebook learned by the reference itself,
    gefen.py:4558-4707) and the trajectory a fresh reference optimizer takes
    after loading it (gefen.py:5456-5707) and stepping the remaining grads
    (ckpt_<name>.npz).  The .pt holds only tensors, numbers, strings and
    containers, so tests load it with torch.load(weights_only=True)."""
    import copy
    _ref()
    from gefen import Gefen
    traj_name, pre = CKPT_CASES[name]
    dtype, factored, params, grads, wd, steps = step_case_inputs(traj_name)
    ps = [(n, torch.nn.Parameter(t.clone())) for n, t, _ in params]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        opt = Gefen(ps, lr=LR, betas=BETAS, eps=EPS, weight_decay=wd, fused=False, factored_v_2d=factored)
    for step_grads in grads[:pre]:
        for (_, p), gv in zip(ps, step_grads):
            p.grad = gv.clone()
        opt.step()
    sd = copy.deepcopy(opt.state_dict())
    torch.save(sd, os.path.join(HERE, "ckpt_%s.pt" % name))
    torch.load(os.path.join(HERE, "ckpt_%s.pt" % name), weights_only=True)  # loadable without unpickling code
    out = {"pre": np.int64(pre), "steps": np.int64(steps), "factored": np.int64(factored), "wd": np.float64(wd)}
    for n, p in ps:
        out["p%d_%s" % (pre, n)] = _f32(p)
    # resume: fresh params holding the trained values, fresh optimizer, load, step on
    ps2 = [(n, torch.nn.Parameter(p.detach().clone())) for n, p in ps]
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        opt2 = Gefen(ps2, lr=LR, betas=BETAS, eps=EPS, weight_decay=wd, fused=False, factored_v_2d=factored)
        opt2.load_state_dict(copy.deepcopy(sd))
    for s in range(pre + 1, steps + 1):
        for (n, p), gv in zip(ps2, grads[s - 1]):
            p.grad = gv.clone()
            out["g%d_%s" % (s, n)] = _f32(gv)
        opt2.step()
        for n, p in ps2:
            st = opt2.state[p]
            out["p%d_%s" % (s, n)] = _f32(p)
            out["idx%d_%s" % (s, n)] = st["m_codebook"].numpy().reshape(-1).copy()
            out["mag%d_%s" % (s, n)] = _f32(st["m_magnitude"]).reshape(-1)
            for key in ("v_row", "v_col", "vmean"):
                if key in st:
                    out["%s%d_%s" % (key, s, n)] = _f32(st[key]).reshape(-1)
    out["global_step"] = np.int64(opt2.state_dict()["gefen_global_step"])
    _save("ckpt_%s.npz" % name, **out)


CASES = {"nearest": case_nearest, "lut": case_lut, "dp": case_dp,
         "learn": case_learn, "period": case_period, "config1": case_config1}
for _n in STEP_CASES:
    CASES["step_" + _n] = (lambda n=_n: case_step(n))
CASES["muon_ns"] = case_muon_ns
for _n in MUON_CASES:
    CASES[_n] = (lambda n=_n: case_muon(n))
CASES["hybrid"] = case_hybrid
for _n in CKPT_CASES:
    CASES["ckpt_" + _n] = (lambda n=_n: case_checkpoint(n))


def main(argv):
    names = argv or [n for n in CASES if n != "config1"]
    for n in names:
        t0 = time.time()
        print("case", n, flush=True)
        CASES[n]()
        print("case", n, "done %.1fs" % (time.time() - t0), flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
