"""The tensor-lr read of Gefen._lr_scalar (reference gefen.py:1530-1555) on
the host: a device lr is read once per (tensor, _version), so a constant lr
costs one read, an in-place scheduler update (which bumps _version) one more,
and a fresh tensor is read afresh; nothing lands in param_groups or the
state_dict.  A CPU tensor stands in for the device lr here."""
import torch

from gefen import Gefen


class _ItemCount:
    def __enter__(self):
        self.n = 0
        self._orig = torch.Tensor.item

        def counted(t):
            self.n += 1
            return self._orig(t)
        torch.Tensor.item = counted
        return self

    def __exit__(self, *exc):
        torch.Tensor.item = self._orig


def _opt(lr):
    return Gefen([("w", torch.nn.Parameter(torch.zeros(8, 8))), ("b", torch.nn.Parameter(torch.zeros(8)))], lr=lr)


def test_float_lr_reads_nothing():
    opt = _opt(1e-3)
    with _ItemCount() as c:
        for _ in range(5):
            assert opt._lr_scalar(opt.param_groups[0]) == 1e-3
    assert c.n == 0


def test_constant_tensor_lr_is_read_once():
    lr = torch.tensor(2e-3)
    opt = _opt(lr)
    with _ItemCount() as c:
        for _ in range(10):
            opt._lr_scalar(opt.param_groups[0])
    assert c.n == 1
    assert opt._lr_scalar(opt.param_groups[0]) == float(torch.tensor(2e-3))


def test_inplace_update_is_seen():
    lr = torch.tensor(1e-3)
    opt = _opt(lr)
    first = opt._lr_scalar(opt.param_groups[0])
    lr.mul_(0.5)  # an in-place scheduler step: _version moves
    with _ItemCount() as c:
        second = opt._lr_scalar(opt.param_groups[0])
        again = opt._lr_scalar(opt.param_groups[0])
    assert c.n == 1
    assert second == again == float(torch.tensor(1e-3) * 0.5) and second != first


def test_fresh_tensor_is_read_and_cache_holds_one_slot():
    opt = _opt(torch.tensor(1e-3))
    for k in range(5):
        opt.param_groups[0]["lr"] = torch.tensor(1e-3 * (k + 1))
        assert opt._lr_scalar(opt.param_groups[0]) == float(torch.tensor(1e-3 * (k + 1)))
    assert isinstance(opt._lr_scalar_cache, tuple) and len(opt._lr_scalar_cache) == 3


def test_cache_not_in_param_groups_or_state_dict():
    opt = _opt(torch.tensor(1e-3))
    opt._lr_scalar(opt.param_groups[0])
    sd = opt.state_dict()
    assert all("_lr_scalar_cache" not in g for g in sd["param_groups"])
    assert "_lr_scalar_cache" not in sd
