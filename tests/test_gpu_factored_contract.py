"""Factored second-moment contract as the reference checks it on a GPU
(tests/test_gefen_factored_v.py there): the state layout and the factored
default, bounded transient memory of a step, a 600,000 x 8 tall matrix's row
and column EMAs against torch, and a checkpoint saved with
factored_v_2d=False resuming under the factored default (v_row / v_col
created lazily, the EMA's bias correction on its own age)."""
import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch.device("cuda", 0)


def test_state_layout_and_factored_default(dev):
    from gefen import Gefen
    torch.manual_seed(3)
    p = nn.Parameter((torch.randn(768, 512, device=dev) * 0.02).bfloat16())
    opt = Gefen([("w", p)], lr=1e-3, factored_v_2d=True, weight_decay=0.1)
    for _ in range(2):
        p.grad = torch.randn(768, 512, device=dev).bfloat16() * 1e-3
        opt.step()
    st = next(iter(opt.state.values()))
    assert st["v_row"].dtype == torch.float32 and tuple(st["v_row"].shape) == (768,)
    assert st["v_col"].dtype == torch.float32 and tuple(st["v_col"].shape) == (512,)
    assert "vmean" not in st
    for factored, has in ((None, "v_row"), (False, "vmean")):
        q = nn.Parameter((torch.randn(64, 32, device=dev) * 0.02).bfloat16())
        kw = {} if factored is None else {"factored_v_2d": factored}
        o = Gefen([("w", q)], lr=1e-3, **kw)
        q.grad = torch.randn(64, 32, device=dev).bfloat16() * 1e-3
        o.step()
        s = next(iter(o.state.values()))
        assert has in s and ({"v_row", "vmean"} - {has}).isdisjoint(s)


def test_transient_memory_of_a_step_is_bounded(dev):
    from gefen import Gefen
    shape = (4096, 4096)
    p = nn.Parameter((torch.randn(*shape, device=dev) * 0.02).bfloat16())
    opt = Gefen([("w", p)], lr=1e-3)
    p.grad = torch.randn(*shape, device=dev).bfloat16() * 1e-3
    opt.step()
    p.grad = torch.randn(*shape, device=dev).bfloat16() * 1e-3
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    opt.step()
    torch.cuda.synchronize()
    extra = torch.cuda.max_memory_allocated() - base
    assert extra < 0.35 * shape[0] * shape[1] * 4, extra


def test_tall_matrix_row_and_column_emas(dev):
    from gefen import Gefen
    rows, cols = 600_000, 8
    torch.manual_seed(9)
    p = nn.Parameter((torch.randn(rows, cols, device=dev) * 0.02).bfloat16())
    opt = Gefen([("w", p)], lr=1e-3)
    g = torch.randn(rows, cols, device=dev).bfloat16() * 1e-3
    p.grad = g.clone()
    opt.step()
    torch.cuda.synchronize()
    st = next(iter(opt.state.values()))
    assert torch.allclose(st["v_row"], g.float().square().mean(dim=1) * (1 - 0.999), rtol=1e-4, atol=1e-12)
    assert torch.allclose(st["v_col"], g.float().square().mean(dim=0) * (1 - 0.999), rtol=1e-4, atol=1e-12)
    assert torch.isfinite(p).all()


def test_block_checkpoint_resumes_under_the_factored_default(dev):
    from gefen import Gefen
    torch.manual_seed(5)
    p = nn.Parameter((torch.randn(96, 64, device=dev) * 0.02).bfloat16())
    old = Gefen([("w", p)], lr=1e-3, factored_v_2d=False)
    torch.manual_seed(6)
    for _ in range(5):
        p.grad = torch.randn(96, 64, device=dev).bfloat16() * 1e-3
        old.step()
    sd = old.state_dict()
    torch.manual_seed(5)
    p2 = nn.Parameter((torch.randn(96, 64, device=dev) * 0.02).bfloat16())
    new = Gefen([("w", p2)], lr=1e-3)
    new.load_state_dict(sd)
    torch.manual_seed(7)
    for _ in range(3):
        p2.grad = torch.randn(96, 64, device=dev).bfloat16() * 1e-3
        new.step()
    torch.cuda.synchronize()
    st = next(iter(new.state.values()))
    assert tuple(st["v_row"].shape) == (96,) and st["factored_step"] == 3
    assert st["step"] == 8
    assert torch.isfinite(p2).all()
