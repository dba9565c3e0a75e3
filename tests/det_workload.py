"""The deterministic=True workload of tests/test_gpu_deterministic.py as a
module and a script (test helper): `python tests/det_workload.py OUT.npz
factored|block` runs it in a fresh process on cuda:0 and writes every state
tensor and parameter after every step, as raw bytes, to OUT.npz."""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

SPECS = [("w2d", (96, 128)), ("big1d", (1 << 21,)), ("odd1d", (99999,)), ("fine1d", (122880,)),
         ("wT", (64, 96))]
PERIODS = {"big1d": 1 << 19, "odd1d": 11111, "fine1d": 40, "w2d": 768, "wT": 768}


def _bits(t):
    """The tensor's bytes in logical order (a bitwise snapshot)."""
    return t.detach().contiguous().clone().reshape(-1).view(torch.uint8)


def run(dev, factored, steps=4):
    """Four seeded steps of a mixed bf16 set (a 2D weight, a transposed view,
    1D tensors whose blocks span many stats workgroups, several blocks per
    wave, and P % 8 != 0); returns one {name: {key: bytes}} per step."""
    from gefen import Gefen
    gen = torch.Generator().manual_seed(4)
    params = []
    for name, shape in SPECS:
        data = (torch.randn(*shape, generator=gen) * 0.02).to(torch.bfloat16)
        if name == "wT":
            p = torch.nn.Parameter(data.t().contiguous().to(dev).t())
        else:
            p = torch.nn.Parameter(data.to(dev))
        params.append((name, p))
    opt = Gefen(params, lr=1e-3, betas=(0.9, 0.999), weight_decay=0.01, factored_v_2d=factored,
                deterministic=True)
    for name, p in params:
        opt.state[p]["automatic_period"] = PERIODS[name]
    cb = np.load(os.path.join(HERE, "golden", "learn.npz"))["cb"]
    opt._gefen_codebook = torch.from_numpy(cb).float().to(dev)
    snaps = []
    for s in range(steps):
        for name, p in params:
            g = (torch.randn(*p.shape, generator=gen) * 10 ** (-3 + s % 2)).to(torch.bfloat16)
            p.grad = g.t().contiguous().to(dev).t() if name == "wT" else g.to(dev)
        opt.step()
        torch.cuda.synchronize()
        snap = {}
        for name, p in params:
            st = opt.state[p]
            snap[name] = {k: _bits(v) for k, v in st.items() if torch.is_tensor(v) and not k.startswith("_")}
            snap[name]["p"] = _bits(p)
        snaps.append(snap)
    return snaps


def main(argv):
    out, mode = argv[1], argv[2]
    for path in (ROOT, os.path.join(ROOT, "gefen-x_amd")):
        if path not in sys.path:
            sys.path.insert(0, path)
    print("det_workload: pid %d, %s" % (os.getpid(), mode), flush=True)
    snaps = run(torch.device("cuda", 0), mode == "factored")
    arrays = {"s%d/%s/%s" % (s, name, k): v.cpu().numpy() for s, snap in enumerate(snaps)
              for name, kv in snap.items() for k, v in kv.items()}
    np.savez(out, **arrays)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))
