"""Muon/backup routing (reference params.py) and the hybrid's argument
checks; CPU only, no kernel calls."""
import pytest
import torch
import torch.nn as nn

from gefen.params import DEFAULT_BACKUP_SUBSTRINGS, is_muon_param, split_params_for_muon, validate_split


class Tiny(nn.Module):
    def __init__(self, tie=True):
        super().__init__()
        self.shared = nn.Embedding(11, 8)          # matches no substring: caught by module type
        self.proj = nn.Linear(8, 16)
        self.norm = nn.LayerNorm(16)
        self.lm_head = nn.Linear(16, 11, bias=False)
        self.frozen = nn.Linear(8, 8)
        self.frozen.weight.requires_grad_(False)
        self.frozen.bias.requires_grad_(False)
        if tie:
            self.head2 = nn.Linear(8, 11, bias=False)
            self.head2.weight = self.shared.weight  # tied to the embedding


def test_split_routes_by_shape_name_and_module_type():
    muon, backup = split_params_for_muon(Tiny())
    assert [n for n, _ in muon] == ["proj.weight"]
    names = {n for n, _ in backup}
    assert {"shared.weight", "proj.bias", "norm.weight", "norm.bias", "lm_head.weight"} <= names
    assert not any(n.startswith("frozen") for n in names)


def test_is_muon_param_rules():
    w = torch.zeros(4, 4)
    assert is_muon_param("layers.0.q_proj.weight", w)
    assert not is_muon_param("model.embed_tokens.weight", w)
    assert not is_muon_param("score.weight", w)
    assert not is_muon_param("layers.0.norm.weight", torch.zeros(4))
    assert "embed" in DEFAULT_BACKUP_SUBSTRINGS


def test_validate_split_rejects_bad_splits():
    a, b = nn.Parameter(torch.zeros(2, 2)), nn.Parameter(torch.zeros(2))
    with pytest.raises(ValueError, match="BOTH"):
        validate_split([("a", a)], [("a2", a)])
    with pytest.raises(ValueError, match="Duplicate parameter name"):
        validate_split([("x", a)], [("X", b)])
    with pytest.raises(ValueError, match="Duplicate parameter object"):
        validate_split([("a", a), ("c", a)], [])
    with pytest.raises(TypeError):
        validate_split([a], [])
    m = Tiny()
    muon, backup = split_params_for_muon(m)
    with pytest.raises(ValueError, match="neither"):
        validate_split(muon, backup[:-1], model=m)
    validate_split(muon, backup, model=m)


def test_ns_schedule_normalisation():
    from gefen.gefen_muon import NS_SCHEDULE_3STEP, _normalize_ns_schedule
    assert _normalize_ns_schedule((1.0, 2.0, 3.0), 4) == [(1.0, 2.0, 3.0)] * 4
    assert _normalize_ns_schedule(NS_SCHEDULE_3STEP, 99) == NS_SCHEDULE_3STEP
    with pytest.raises(ValueError):
        _normalize_ns_schedule((1.0, 2.0, 3.0), 0)
    with pytest.raises(ValueError):
        _normalize_ns_schedule([(1.0, 2.0)], 5)


def test_adjust_lr_ratio():
    from gefen.gefen_muon import _adjust_lr_ratio
    assert _adjust_lr_ratio(None, (4096, 1024)) == 2.0
    assert _adjust_lr_ratio("original", (1024, 4096)) == 1.0
    assert abs(_adjust_lr_ratio("match_rms_adamw", (14336, 4096)) - 0.2 * 14336 ** 0.5) < 1e-12
