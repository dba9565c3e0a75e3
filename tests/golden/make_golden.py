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


CASES = {"nearest": case_nearest, "lut": case_lut, "dp": case_dp,
         "learn": case_learn, "period": case_period, "config1": case_config1}
for _n in STEP_CASES:
    CASES["step_" + _n] = (lambda n=_n: case_step(n))


def main(argv):
    names = argv or [n for n in CASES if n != "config1"]
    for n in names:
        t0 = time.time()
        print("case", n, flush=True)
        CASES[n]()
        print("case", n, "done %.1fs" % (time.time() - t0), flush=True)


if __name__ == "__main__":
    main(sys.argv[1:])
