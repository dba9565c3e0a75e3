"""gefenx_factored_update_noalloc against gefenx_factored_update through the
C ABI: two calls in a row on one GPU, the second with a smaller parameter
(so the static scratch holds the first call's contents when the second
starts), each compared bit for bit with the workspace entry point on the
same inputs: parameters, indices, magnitudes, v_row and v_col.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def _state(rows, cols, period, dtype, seed, dev):
    gen = torch.Generator().manual_seed(seed)
    nb = rows * cols // period
    return {
        "p": (torch.randn(rows, cols, generator=gen) * 0.02).to(dtype).to(dev),
        "g": (torch.randn(rows, cols, generator=gen) * 1e-3).to(dtype).to(dev),
        "idx": torch.randint(0, 256, (nb, period), generator=gen, dtype=torch.uint8).to(dev),
        "mag": (torch.rand(nb, 1, generator=gen) * 1e-3).to(dev),
        "vr": (torch.rand(rows, generator=gen) * 1e-6).to(dev),
        "vc": (torch.rand(cols, generator=gen) * 1e-6).to(dev),
    }


def _call(lib, fused, st, period, qt, noalloc, step):
    from gefen.kernels import _native
    rows, cols = st["p"].shape
    bc1, bc2 = 1 - 0.9 ** step, 1 - 0.999 ** step
    args = [st["p"].data_ptr(), st["g"].data_ptr(), fused._dtype_code(st["p"].dtype), rows, cols,
            st["p"].stride(0), st["p"].stride(1), st["g"].stride(0), st["g"].stride(1),
            st["idx"].data_ptr(), st["mag"].data_ptr(), st["vr"].data_ptr(), st["vc"].data_ptr(), period,
            qt.data_ptr(), 0.9, 0.999, 6e-5, 1e-8, 1.0 / bc2, 1.0 / bc1, 1.0 - 6e-5 * 0.01, 0, 0, None, None]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.gefenx_factored_update_noalloc(*args, stream)
    else:
        nbytes = int(lib.gefenx_workspace_bytes(_native.WS_FACTORED, rows, cols, rows * cols // period))
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=st["p"].device)
        rc = lib.gefenx_factored_update(*args, ws.data_ptr(), ws.numel(), stream)
    _native.check(rc, "noalloc test")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(dev, dtype):
    from gefen.kernels import _native
    from gefen.kernels import automatic_gefen_fused as fused
    lib = _native.load()
    cb = torch.from_numpy(np.load(os.path.join(GOLD, "learn.npz"))["cb"]).float().to(dev)
    qt = fused.quant_table(cb, dtype)
    # second call smaller than the first; its block count (32 shards x 64 of
    # them) differs, so stale maxima of the first call would show
    for call, (rows, cols, period) in enumerate([(1024, 4096, 4096), (384, 640, 3840)]):
        print("noalloc call %d %s [%d, %d] P=%d" % (call, dtype, rows, cols, period), flush=True)
        a = _state(rows, cols, period, dtype, 100 + call, dev)
        b = {k: v.clone() for k, v in a.items()}
        _call(lib, fused, a, period, qt, noalloc=False, step=call + 1)
        _call(lib, fused, b, period, qt, noalloc=True, step=call + 1)
        torch.cuda.synchronize()
        for k in ("p", "idx", "mag", "vr", "vc"):
            x, y = a[k].contiguous().view(-1), b[k].contiguous().view(-1)
            assert torch.equal(x.view(torch.uint8) if x.dtype != torch.uint8 else x,
                               y.view(torch.uint8) if y.dtype != torch.uint8 else y), (call, k)
