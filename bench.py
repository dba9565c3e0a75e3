#!/usr/bin/env python
"""Benchmark: one Gefen optimizer step (opt.step()) on MI355X.

Workload: a Llama-3-8B-shaped bf16 parameter set --
32 layers x {q 4096x4096, k/v 1024x4096, o 4096x4096, gate/up 14336x4096,
down 4096x14336, two 4096 RMSNorm vectors} plus a 128256x4096 embedding and a
128256x4096 lm_head: 290 tensors, 8,030,257,152 params.  Plain Gefen with
factored_v_2d, lr 6e-5, betas (0.9, 0.999), eps 1e-8, weight decay 0.01.
Params ~ N(0, 0.02); grads per tensor ~ N(0, sigma), sigma log-uniform in
[1e-4, 1e-2], all from fixed seeds (synthetic data).  The first warm-up step
runs the period search and learns the codebook; momentum state then comes from
the remaining seeded warm-up steps (fresh grads each); the timed steps reuse
the last grads, resident in HBM.

One JSON line on stdout: params/s of the whole step plus a `roofline` object
for the dominant kernel (the fused apply: algorithmic bytes / its HIP-event
time over the timed region) and a `cpu_baseline` object (the C oracle of the
reference's CPU step, single-threaded, on a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "gefen-x_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBPS = 8000.0
METRIC = "params updated/sec per opt.step + achieved HBM GB/s vs peak, Llama-3-8B shapes"


def llama3_8b_shapes():
    shapes = [("model.embed_tokens.weight", (128256, 4096))]
    for i in range(32):
        pre = "model.layers.%d." % i
        shapes += [
            (pre + "self_attn.q_proj.weight", (4096, 4096)),
            (pre + "self_attn.k_proj.weight", (1024, 4096)),
            (pre + "self_attn.v_proj.weight", (1024, 4096)),
            (pre + "self_attn.o_proj.weight", (4096, 4096)),
            (pre + "mlp.gate_proj.weight", (14336, 4096)),
            (pre + "mlp.up_proj.weight", (14336, 4096)),
            (pre + "mlp.down_proj.weight", (4096, 14336)),
            (pre + "input_layernorm.weight", (4096,)),
            (pre + "post_attention_layernorm.weight", (4096,)),
        ]
    shapes.append(("lm_head.weight", (128256, 4096)))
    return shapes


def _log(*a):
    print(*a, file=sys.stderr, flush=True)


def make_params(torch, shapes, device, seed=0):
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    params = []
    for name, shape in shapes:
        p = torch.empty(shape, dtype=torch.bfloat16, device=device)
        p.normal_(0.0, 0.02, generator=gen)
        params.append((name, torch.nn.Parameter(p)))
    return params


def fill_grads(torch, params, step_seed, device):
    gen = torch.Generator(device=device)
    gen.manual_seed(10_000 + step_seed)
    host = torch.Generator().manual_seed(20_000 + step_seed)
    for _, p in params:
        sigma = 10.0 ** float(torch.empty(1).uniform_(-4.0, -2.0, generator=host))
        if p.grad is None:
            p.grad = torch.empty_like(p)
        p.grad.normal_(0.0, sigma, generator=gen)


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gefen_step_llama3_8b_traffic.json")
APPLY_KERNEL = "k_mt_apply<2, 0, false, true>"  # bf16, factored, nearest rounding, contiguous fast path
KERNEL_SOURCES = ("gefenx_update.hip", "gefenx_device.h", "gefenx_common.h")


def _kernel_source_sha():
    """sha256 over the sources of the step kernels: a committed traffic
    measurement counts only for the kernels it was taken on."""
    import hashlib
    h = hashlib.sha256()
    for name in KERNEL_SOURCES:
        with open(os.path.join(ROOT, "gefen-x_amd", "csrc", name), "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def _measured_traffic(key="apply_traffic_bytes_per_launch"):
    """HBM bytes from the committed rocprofv3 PMC passes (FETCH_SIZE x its
    copy-calibrated scale + WRITE_SIZE x its scale): per launch of the
    factored apply by default, or `key` (e.g. the whole step's bytes); None
    when no measurement is committed or it was taken on other kernel sources."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    if t.get("kernel_source_sha256") != _kernel_source_sha():
        _log("bench: %s was measured on other kernel sources; traffic reported as null" %
             os.path.relpath(TRAFFIC_FILE, ROOT))
        return None
    try:
        return float(t[key])
    except (KeyError, ValueError, TypeError):
        return None


def _pmc_avg(path, counter, pattern):
    """Average per dispatch of `counter` over the kernels whose name contains
    `pattern`, from a rocprofv3 --pmc csv (a file, or a directory searched for
    *counter_collection.csv)."""
    import csv
    import glob
    files = [path] if os.path.isfile(path) else sorted(glob.glob(os.path.join(path, "**", "*counter_collection.csv"),
                                                                 recursive=True))
    vals = []
    for fn in files:
        with open(fn) as f:
            for r in csv.DictReader(f):
                if r["Counter_Name"] == counter and pattern in r["Kernel_Name"]:
                    vals.append(float(r["Counter_Value"]))
    if not vals:
        raise SystemExit("no %s rows for kernels matching %r under %s" % (counter, pattern, path))
    return sum(vals) / len(vals), len(vals)


def write_traffic(fetch, write, copy_fetch, copy_write):
    """Combine the four PMC passes (the bench's apply kernel: FETCH_SIZE,
    WRITE_SIZE; the --calibrate-copy run: FETCH_SIZE, WRITE_SIZE) into the
    committed traffic figure.  Counters are KiB per dispatch; each is scaled
    so that the plain 1 GiB copy reads and writes exactly 1 GiB."""
    copy_bytes = float(1 << 30)
    cf, _ = _pmc_avg(copy_fetch, "FETCH_SIZE", "copyBuffer")
    cw, _ = _pmc_avg(copy_write, "WRITE_SIZE", "copyBuffer")
    sf, sw = copy_bytes / (cf * 1024.0), copy_bytes / (cw * 1024.0)
    af, nf = _pmc_avg(fetch, "FETCH_SIZE", APPLY_KERNEL)
    aw, nw = _pmc_avg(write, "WRITE_SIZE", APPLY_KERNEL)
    # the other launches of the steady-state step (one of each per step)
    step = af * 1024.0 * sf + aw * 1024.0 * sw
    others = {}
    for pat in ("k_mt_factored_stats", "k_mt_finalize", "k_mt_mean"):
        f, _ = _pmc_avg(fetch, "FETCH_SIZE", pat)
        w, _ = _pmc_avg(write, "WRITE_SIZE", pat)
        others[pat] = f * 1024.0 * sf + w * 1024.0 * sw
        step += others[pat]
    out = {"kernel": APPLY_KERNEL, "dispatches": [nf, nw],
           "fetch_kib_per_dispatch": af, "write_kib_per_dispatch": aw,
           "copy_fetch_kib": cf, "copy_write_kib": cw, "fetch_scale": sf, "write_scale": sw,
           "apply_read_bytes_per_launch": af * 1024.0 * sf, "apply_write_bytes_per_launch": aw * 1024.0 * sw,
           "apply_traffic_bytes_per_launch": af * 1024.0 * sf + aw * 1024.0 * sw,
           "other_launch_bytes": others, "step_traffic_bytes": step,
           "kernel_source_sha256": _kernel_source_sha()}
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    print(json.dumps(out))
    return 0


def _cpu_cores_and_model():
    """Cores this process may run on (sched_getaffinity, capped by
    OMP_NUM_THREADS when the box sets it) and the CPU model string."""
    cores = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        cores = min(cores, int(omp))
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return cores, model


LLAMA_CLASS_COUNTS = {"embed": 1, "lm_head": 1, "q_proj": 32, "k_proj": 32, "v_proj": 32, "o_proj": 32,
                      "gate_proj": 32, "up_proj": 32, "down_proj": 32, "layernorm": 64}


def _class_of(name):
    if "embed_tokens" in name:
        return "embed"
    if name.startswith("lm_head"):
        return "lm_head"
    for c in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"):
        if c in name:
            return c
    return "layernorm"


def cpu_baseline(torch, params=None, opt=None):
    """The CPU step of BASELINE.md, timed on this box's host cores: the C
    oracle (the build's restatement of the reference's decomposed fused=False
    step, pinned to the reference's golden trajectories), threaded over every
    core this process may use (its parallel loops keep each element's order,
    so the results do not depend on the thread count).

    - W 4096x4096 + b 4096 fp32 from the config-1 seeds, 10 steps
      (step 1 includes the period search and the exact-DP codebook), each
      timed; the median is reported.
    - one tensor of every class of the Llama-3-8B set -- the GPU
      run's own parameters, grads, searched periods, codebook and state,
      copied to the host -- stepped once each; the full-set CPU step time is
      the sum over classes of (tensors in the class x that tensor's time),
      and `value` is the set's params over that time."""
    import numpy as np
    from oracle import oracle as orc
    cores, model = _cpu_cores_and_model()
    orc.set_threads(cores)
    out = {"unit": "params/s", "cores": cores, "cpu_model": model, "kind": "port"}
    try:
        # configs[0]
        gen = torch.Generator().manual_seed(0)
        w = (torch.randn(4096, 4096, generator=gen) * 0.02).numpy()
        b = (torch.randn(4096, generator=gen) * 0.02).numpy()
        times = []
        st = None
        for s in range(1, 11):
            gt = torch.Generator().manual_seed(1000 + s)
            gw = (torch.randn(4096, 4096, generator=gt) * 1e-3).numpy()
            gb = (torch.randn(4096, generator=gt) * 1e-3).numpy()
            t0 = time.perf_counter()
            if st is None:
                pw, pb = orc.resolve_period(gw, gw.shape), orc.resolve_period(gb, gb.shape)
                cb = orc.learn_codebook([(gw, pw), (gb, pb)])
                st = {"iw": np.zeros(gw.size, np.uint8), "mw": np.zeros(gw.size // pw, np.float32),
                      "vr": np.zeros(4096, np.float32), "vc": np.zeros(4096, np.float32),
                      "ib": np.zeros(gb.size, np.uint8), "mb": np.zeros(gb.size // pb, np.float32),
                      "vm": np.zeros(gb.size // pb, np.float32)}
            kw = dict(beta1=0.9, beta2=0.999, lr=6e-5, eps=1e-8, bc1=1 - 0.9 ** s, bc2=1 - 0.999 ** s, wd=0.01)
            w, st["iw"], st["mw"], st["vr"], st["vc"] = orc.factored_step(
                w, gw, st["iw"], st["mw"], st["vr"], st["vc"], pw, cb, orc.F32, **kw)
            b, st["ib"], st["mb"], st["vm"] = orc.block_step(b, gb, st["ib"], st["mb"], st["vm"], pb, cb, orc.F32,
                                                             **kw)
            times.append(time.perf_counter() - t0)
        c1_ms = sorted(times)[len(times) // 2] * 1e3
        out["config0_step_ms_median"] = c1_ms
        out["config0_step1_ms"] = times[0] * 1e3
        out["config0_params_per_s"] = (4096 * 4096 + 4096) / (c1_ms / 1e3)
        # configs[1], one tensor per class
        if params is not None and opt is not None:
            cb = opt._gefen_codebook.detach().cpu().numpy()
            seen = {}
            for name, p in params:
                cls = _class_of(name)
                if cls in seen:
                    continue
                stt = opt.state[p]
                per = int(stt["automatic_period"])
                step = int(stt["step"]) + 1
                kw = dict(beta1=0.9, beta2=0.999, lr=6e-5, eps=1e-8, bc1=1 - 0.9 ** step, bc2=1 - 0.999 ** step,
                          wd=0.01)
                pn = p.detach().float().cpu().numpy()
                gn = p.grad.detach().float().cpu().numpy()
                idx = stt["m_codebook"].cpu().numpy().reshape(-1)
                mag = stt["m_magnitude"].cpu().numpy().reshape(-1)
                t0 = time.perf_counter()
                if "v_row" in stt:
                    orc.factored_step(pn, gn, idx, mag, stt["v_row"].cpu().numpy(), stt["v_col"].cpu().numpy(),
                                      per, cb, orc.BF16, **kw)
                else:
                    orc.block_step(pn, gn, idx, mag, stt["vmean"].cpu().numpy().reshape(-1), per, cb, orc.BF16,
                                   **kw)
                seen[cls] = (time.perf_counter() - t0, p.numel())
                del pn, gn, idx, mag
            full_s = sum(LLAMA_CLASS_COUNTS[c] * t for c, (t, _) in seen.items())
            n_full = sum(LLAMA_CLASS_COUNTS[c] * n for c, (_, n) in seen.items())
            out["value"] = n_full / full_s
            out["config1_step_s_estimate"] = full_s
            out["config1_class_ms"] = {c: round(t * 1e3, 2) for c, (t, _) in seen.items()}
            out["sample"] = ("configs[1]: one oracle step of one tensor per class of the Llama-3-8B set (the GPU "
                             "run's tensors, periods, codebook and state), scaled by the class counts to the full "
                             "8.03e9-param set; configs[0]: 10 steps of 4096x4096+4096 fp32, median")
        else:
            out["value"] = out["config0_params_per_s"]
            out["sample"] = "configs[0]: 10 steps of 4096x4096+4096 fp32, median"
    finally:
        orc.set_threads(1)
    return out


def bench_muon(args):
    """GefenMuonHybrid on the Llama-3-8B layer stack
    (224 hidden matrices -> quantised momentum + 5-step standard Newton-Schulz
    in bf16 on MFMA; 64 norms + embedding + lm_head -> block-vmean Gefen
    backup).  bf16 params, grads N(0, 1e-3).  Reports the whole step and the
    Newton-Schulz GEMMs' throughput: `achieved` counts the algorithmic FLOPs
    of three full products per iteration; `executed_tflops` /
    `mfma_utilisation` count what the MFMAs run (the two symmetric products
    compute only their lower-triangle tiles)."""
    import torch
    from gefen import GefenMuonHybrid
    from gefen.kernels import _native
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    shapes = llama3_8b_shapes()
    params = make_params(torch, shapes, dev)
    from gefen.params import is_muon_param
    muon = [(n, p) for n, p in params if is_muon_param(n, p)]
    backup = [(n, p) for n, p in params if not is_muon_param(n, p)]
    n_params = sum(p.numel() for _, p in params)
    _log("bench muon: %d muon matrices, %d backup tensors, %d params" % (len(muon), len(backup), n_params))
    opt = GefenMuonHybrid(muon, backup, lr=1e-3, weight_decay=0.01, ns_schedule="standard", ns_steps=5)
    gen = torch.Generator(device=dev)
    for w in range(max(1, args.warmup)):
        gen.manual_seed(30_000 + w)
        for _, p in params:
            if p.grad is None:
                p.grad = torch.empty_like(p)
            p.grad.normal_(0.0, 1e-3, generator=gen)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        opt.step()
        torch.cuda.synchronize()
        _log("bench muon: warm-up step %d %.2f s" % (w, time.perf_counter() - t0))
    lib = _native.load()
    lib.gefenx_profile_reset()
    lib.gefenx_profile_enable(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        opt.step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    lib.gefenx_profile_enable(0)
    ns_ms, ns_n, _, ns_flops = _native.profile_read(_native.K_NS_GEMM)
    mom_ms, mom_n, mom_bytes, _ = _native.profile_read(_native.K_MOMENTUM)
    lib.gefenx_profile_reset()
    ms_step = elapsed * 1e3 / args.steps
    tflops = ns_flops / (ns_ms / 1e3) / 1e12 if ns_ms > 0 else 0.0
    # FLOPs the MFMAs actually execute: G = XX^T and GG^T are symmetric, so
    # only their lower-triangle 128 x 128 tiles run ((T+1)/2T of the tiles)
    executed = 0.0
    for _, p in muon:
        m, n = min(p.shape), max(p.shape)
        t = -(-m // 128)
        tri = (t + 1) / (2.0 * t)
        executed += 5 * (2.0 * m * m * n * tri + 2.0 * m * m * m * tri + 2.0 * m * m * n)
    exec_tflops = executed / (ns_ms / 1e3 / args.steps) / 1e12 if ns_ms > 0 else 0.0
    out = {
        "metric": METRIC + " (GefenMuonHybrid workload)",
        "value": n_params / (elapsed / args.steps), "unit": "params/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms_step, "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) params, N(0,1e-3) grads)",
        "config": {"workload": "GefenMuonHybrid, Llama-3-8B layer stack: 224 Muon matrices (5-step standard "
                               "Newton-Schulz, bf16 MFMA) + 66 backup tensors", "params": n_params,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": tflops / 2500.0, "traffic": None,
                     "kernel": "k_gemm_big16 / k_gemm_big / k_gemm_dl (Newton-Schulz GEMMs, bf16 MFMA, direct-to-LDS; 256x256 tiles on large grids, 16x16x32 when every tile is full)",
                     "flops_per_step": ns_flops / args.steps, "gemm_ms_per_step": ns_ms / args.steps,
                     "executed_flops_per_step": executed, "executed_tflops": exec_tflops,
                     "mfma_utilisation": exec_tflops / 2500.0},
        "momentum_kernel": {"ms_per_step": mom_ms / args.steps,
                            "GB/s": mom_bytes / (mom_ms / 1e3) / 1e9 if mom_ms > 0 else 0.0},
    }
    print(json.dumps(out), flush=True)
    return 0


def qwen3_4b_shapes():
    """Qwen3-4B (36 layers, hidden 2560, GQA q 4096x2560,
    k/v 1024x2560, o 2560x4096, MLP 9728, q/k-norm 128, vocab 151936 tied)."""
    shapes = [("model.embed_tokens.weight", (151936, 2560))]
    for i in range(36):
        pre = "model.layers.%d." % i
        shapes += [(pre + "self_attn.q_proj.weight", (4096, 2560)), (pre + "self_attn.k_proj.weight", (1024, 2560)),
                   (pre + "self_attn.v_proj.weight", (1024, 2560)), (pre + "self_attn.o_proj.weight", (2560, 4096)),
                   (pre + "self_attn.q_norm.weight", (128,)), (pre + "self_attn.k_norm.weight", (128,)),
                   (pre + "mlp.gate_proj.weight", (9728, 2560)), (pre + "mlp.up_proj.weight", (9728, 2560)),
                   (pre + "mlp.down_proj.weight", (2560, 9728)), (pre + "input_layernorm.weight", (2560,)),
                   (pre + "post_attention_layernorm.weight", (2560,))]
    shapes.append(("model.norm.weight", (2560,)))
    return shapes


def make_qwen_params(torch, dev, seed=0):
    """The Qwen3-4B-shaped bf16 set, N(0, 0.02) from a seed; every 10th 2D
    tensor is a transposed view (.t()) of [C, R] storage."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    params, n2d = [], 0
    for name, shape in qwen3_4b_shapes():
        if len(shape) == 2:
            n2d += 1
            if n2d % 10 == 0:
                st = torch.empty(shape[1], shape[0], dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=gen)
                params.append((name, torch.nn.Parameter(st.t())))
                continue
        params.append((name, torch.nn.Parameter(
            torch.empty(shape, dtype=torch.bfloat16, device=dev).normal_(0.0, 0.02, generator=gen))))
    return params


def fill_qwen_grads(torch, params, step_seed, dev):
    """Grads 1e-3 * StudentT(nu=3) from a seed, drawn as z * sqrt(3 / chi2_3)
    (chi2_3 the sum of three squared normals); a transposed-view parameter
    gets a grad of the same layout."""
    gen = torch.Generator(device=dev).manual_seed(50_000 + step_seed)
    for _, p in params:
        shape = tuple(p.shape)
        z = torch.empty(shape, dtype=torch.float32, device=dev).normal_(generator=gen)
        chi2 = torch.zeros(shape, dtype=torch.float32, device=dev)
        for _ in range(3):
            chi2.add_(torch.empty(shape, dtype=torch.float32, device=dev).normal_(generator=gen).square_())
        g = (z * torch.rsqrt(chi2.div_(3.0)) * 1e-3).to(torch.bfloat16)
        del z, chi2
        if not p.is_contiguous():
            g = g.t().contiguous().t()
        p.grad = g


def bench_qwen(args):
    """the many-tensor launcher on a Qwen3-4B-shaped
    bf16 set (398 tensors, 4,022,468,096 params); 25 of the 253 2D tensors
    (every 10th) are transposed views of [C, R] storage; grads 1e-3 *
    StudentT(nu=3) from a seed; factored_v_2d on, then off.  Reports ms/step,
    launches per step and the host time of opt.step() (launch overhead)."""
    import torch
    from gefen import Gefen
    from gefen.kernels import _native
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    params = make_qwen_params(torch, dev)
    n_params = sum(p.numel() for _, p in params)
    n_views = sum(1 for _, p in params if not p.is_contiguous())
    fill_qwen_grads(torch, params, 0, dev)
    lib = _native.load()
    results = {}
    for factored in (True, False):
        opt = Gefen(params, lr=6e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, factored_v_2d=factored)
        for _ in range(max(1, args.warmup)):
            opt.step()
        torch.cuda.synchronize()
        lib.gefenx_profile_reset()
        lib.gefenx_profile_enable(1)
        t0 = time.perf_counter()
        for _ in range(args.steps):
            opt.step()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        lib.gefenx_profile_enable(0)
        host = 0.0
        for _ in range(5):  # host cost of one call (enqueue only, GPU idle at entry)
            torch.cuda.synchronize()
            h0 = time.perf_counter()
            opt.step()
            host += time.perf_counter() - h0
        torch.cuda.synchronize()
        launches = sum(_native.profile_read(k)[1] for k in (_native.K_STATS, _native.K_FINALIZE, _native.K_APPLY,
                                                             _native.K_BLOCK_STATS, _native.K_BLOCK_APPLY))
        apply_ms, apply_n, apply_b, _ = _native.profile_read(_native.K_APPLY)
        bapply_ms, _, bapply_b, _ = _native.profile_read(_native.K_BLOCK_APPLY)
        lib.gefenx_profile_reset()
        ms = elapsed * 1e3 / args.steps
        results["factored" if factored else "block"] = {
            "ms_per_step": ms, "params_per_s": n_params / (elapsed / args.steps),
            "compulsory_GB_per_s": (apply_b + bapply_b) / args.steps / (ms / 1e3) / 1e9,
            "launches_per_step": launches / args.steps, "host_us_per_call": host * 1e6 / 5}
        _log("bench qwen factored=%s: %s" % (factored, results["factored" if factored else "block"]))
        del opt
        torch.cuda.empty_cache()
    r = results["factored"]
    out = {"metric": METRIC + " (Qwen3-4B many-tensor workload)", "value": r["params_per_s"], "unit": "params/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": r["ms_per_step"],
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
           "data": "synthetic (seeded N(0,0.02) params, 1e-3*StudentT(3) grads)",
           "config": {"workload": "Qwen3-4B-shaped bf16 set, 398 tensors, %d transposed views" % n_views,
                      "params": n_params, "parallelism": "single GPU"},
           "factored_v_2d_on": results["factored"], "factored_v_2d_off": results["block"]}
    print(json.dumps(out), flush=True)
    return 0


def bench_capturable(torch, params, dev, steps, lr=6e-5):
    """capturable=True on the same tensor set: eager stepping, then one
    captured step replayed (device step counters, tensor lr, no host work per
    replay).  Returns ms per step of each and the host time of an eager call."""
    from gefen import Gefen
    lr_t = torch.tensor(lr, device=dev)
    opt = Gefen(params, lr=lr_t, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, factored_v_2d=True,
                capturable=True)
    for _ in range(3):
        opt.step()
    torch.cuda.synchronize()
    host = 0.0
    t0 = time.perf_counter()
    for _ in range(steps):
        h0 = time.perf_counter()
        opt.step()
        host += time.perf_counter() - h0
    torch.cuda.synchronize()
    eager_ms = (time.perf_counter() - t0) * 1e3 / steps
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        opt.step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        opt.step()
    graph.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        graph.replay()
    torch.cuda.synchronize()
    graph_ms = (time.perf_counter() - t0) * 1e3 / steps
    del graph, opt
    torch.cuda.synchronize()
    return {"eager_ms_per_step": eager_ms, "graph_replay_ms_per_step": graph_ms,
            "eager_host_ms_per_call": host * 1e3 / steps, "steps": steps}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-capturable", action="store_true",
                    help="skip the capturable=True eager / graph-replay timing on the headline set")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 1 GiB device copy 4 times (scale for rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE counters)")
    ap.add_argument("--workload", choices=["gefen", "muon", "qwen"], default="gefen",
                    help="gefen: configs[1], the headline Llama-3-8B Gefen step (default); "
                         "muon: configs[3], GefenMuonHybrid with MFMA utilisation; "
                         "qwen: configs[2], the many-tensor Qwen3-4B set, factored on and off")
    ap.add_argument("--traffic-from", nargs=4, metavar=("FETCH", "WRITE", "COPY_FETCH", "COPY_WRITE"),
                    help="write the committed traffic figure from four rocprofv3 --pmc csv outputs (the bench's "
                         "FETCH_SIZE and WRITE_SIZE passes, then --calibrate-copy's) and exit")
    args = ap.parse_args(argv)
    if args.traffic_from:
        return write_traffic(*args.traffic_from)
    if args.calibrate_copy:
        import torch
        src = torch.ones(1 << 29, dtype=torch.int16, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2,
                          "launches": 4}))
        return 0
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build runs the optimizer step on a single GPU "
              "(multi-GPU sharding is a design note, not part of this build); got --gpus %d" % args.gpus,
              file=sys.stderr)
        return 2
    if args.workload == "muon":
        return bench_muon(args)
    if args.workload == "qwen":
        return bench_qwen(args)
    import torch
    from gefen import Gefen
    from gefen.kernels import _native

    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    shapes = llama3_8b_shapes()
    n_params = sum(int(torch.Size(s).numel()) for _, s in shapes)
    _log("bench: %d tensors, %d params on %s" % (len(shapes), n_params, torch.cuda.get_device_name(0)))
    params = make_params(torch, shapes, dev)
    opt = Gefen(params, lr=6e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, factored_v_2d=True)

    t_first = None
    for w in range(max(1, args.warmup)):
        fill_grads(torch, params, w, dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        opt.step()
        torch.cuda.synchronize()
        if w == 0:
            t_first = time.perf_counter() - t0
            periods = sorted({(opt.state[p]["automatic_period"]) for _, p in params})
            _log("bench: step 1 (period search + codebook) %.2f s; periods %s" % (t_first, periods[:12]))
    _log("bench: warmup done")

    lib = _native.load()
    lib.gefenx_profile_reset()
    lib.gefenx_profile_enable(1)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        opt.step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    lib.gefenx_profile_enable(0)
    ms_step = elapsed * 1e3 / args.steps
    value = n_params / (elapsed / args.steps)
    host = 0.0
    for _ in range(5):  # host cost of one eager call (enqueue only)
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        opt.step()
        host += time.perf_counter() - h0
    torch.cuda.synchronize()

    kinds = {}
    for name, kind in (("stats", _native.K_STATS), ("finalize", _native.K_FINALIZE), ("apply", _native.K_APPLY),
                       ("block_stats", _native.K_BLOCK_STATS), ("block_apply", _native.K_BLOCK_APPLY)):
        kinds[name] = _native.profile_read(kind)
    # the block-path vectors ride in the factored launches: no launches of their own
    kinds = {k: v for k, v in kinds.items() if v[1] > 0 or k in ("stats", "finalize", "apply")}
    lib.gefenx_profile_reset()
    # dominant kernel: the factored (2D) apply, one launch per step
    apply_ms, apply_n, apply_bytes, _ = kinds["apply"]
    achieved = apply_bytes / (apply_ms / 1e3) / 1e9 if apply_ms > 0 else 0.0
    step_bytes = (apply_bytes + kinds.get("block_apply", (0, 0, 0.0))[2]) / args.steps  # compulsory bytes per step
    _log("bench: kernel ms per step: " + ", ".join(
        "%s %.3f (%d launches)" % (k, v[0] / args.steps, v[1] // args.steps) for k, v in kinds.items()))
    _log("bench: %.3f ms/step, %.1f GB/s compulsory over the whole step" % (
        ms_step, step_bytes / (ms_step / 1e3) / 1e9))

    moved = _measured_traffic("step_traffic_bytes")
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "params/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) params, N(0,sigma) grads, sigma log-uniform [1e-4,1e-2])",
        "config": {"workload": "Llama-3-8B-shaped bf16 set, plain Gefen, factored_v_2d, 290 tensors",
                   "params": n_params, "lr": 6e-5, "betas": [0.9, 0.999], "eps": 1e-8,
                   "weight_decay": 0.01, "parallelism": "single GPU"},
        "step_hbm_gbps": step_bytes / (ms_step / 1e3) / 1e9,
        "step_frac_of_peak": step_bytes / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBPS,
        # bytes the whole step moves (PMC: stats re-read of grads + indices,
        # partials, finalize, applies) over the step time
        "step_moved_gbps": (moved / (ms_step / 1e3) / 1e9) if moved else None,
        "step_moved_frac_of_peak": (moved / (ms_step / 1e3) / 1e9 / HBM_PEAK_GBPS) if moved else None,
        "kernel_ms_per_step": {k: v[0] / args.steps for k, v in kinds.items()},
        "first_step_s": t_first,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS, "traffic": _measured_traffic(),
                     "kernel": "k_mt_apply<bf16, factored> (fused requantize + apply of the 226 2D tensors)",
                     "algo_bytes_per_launch": apply_bytes / max(1, apply_n),
                     "avg_launch_ms": apply_ms / max(1, apply_n)},
    }
    out["eager_host_ms_per_call"] = host * 1e3 / 5
    if not args.no_cpu_baseline:
        _log("bench: cpu baseline (oracle on the host cores) ...")
        out["cpu_baseline"] = cpu_baseline(torch, params, opt)
        _log("bench: cpu baseline %s" % json.dumps(out["cpu_baseline"]))
    if not args.no_capturable:
        del opt
        _log("bench: capturable eager and graph replay ...")
        out["capturable"] = bench_capturable(torch, params, dev, min(args.steps, 20))
        _log("bench: capturable %s" % json.dumps(out["capturable"]))
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
