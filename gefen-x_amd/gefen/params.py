"""Routing of parameters between Muon and the Gefen backup (reference
params.py:30-187): 2D hidden weight matrices go to Muon; embeddings (by module
type, which also catches tied heads), LM / classifier heads (by name) and every
1D or other-shaped tensor go to the backup."""
from __future__ import annotations

import logging
from typing import Iterable, List, Tuple

import torch
import torch.nn as nn

logger = logging.getLogger(__name__)

# Name substrings routed to the backup (params.py:30-37).
DEFAULT_BACKUP_SUBSTRINGS: Tuple[str, ...] = (
    "embed",
    "wte",
    "wpe",
    "lm_head",
    "classifier",
    "score",
)


def is_muon_param(name: str, param, backup_substrings=DEFAULT_BACKUP_SUBSTRINGS) -> bool:
    """params.py:40-45: a 2D tensor whose name matches no backup substring."""
    if param.ndim != 2:
        return False
    lname = name.lower()
    return not any(sub.lower() in lname for sub in backup_substrings)


def _embedding_param_ids(model: nn.Module) -> set:
    """ids of every nn.Embedding / nn.EmbeddingBag weight (params.py:48-62)."""
    ids = set()
    for module in model.modules():
        if isinstance(module, (nn.Embedding, nn.EmbeddingBag)):
            weight = getattr(module, "weight", None)
            if weight is not None:
                ids.add(id(weight))
    return ids


def split_params_for_muon(
    model: nn.Module,
    backup_substrings: Iterable[str] = DEFAULT_BACKUP_SUBSTRINGS,
) -> Tuple[List[Tuple[str, nn.Parameter]], List[Tuple[str, nn.Parameter]]]:
    """(muon_named, backup_named) of the model's trainable parameters
    (params.py:65-101); frozen parameters are skipped."""
    backup_substrings = tuple(backup_substrings)
    embedding_ids = _embedding_param_ids(model)
    muon: List[Tuple[str, nn.Parameter]] = []
    backup: List[Tuple[str, nn.Parameter]] = []
    for name, p in model.named_parameters():
        if not p.requires_grad:
            continue
        if id(p) not in embedding_ids and is_muon_param(name, p, backup_substrings):
            muon.append((name, p))
        else:
            backup.append((name, p))
    logger.info("split_params_for_muon: %d muon / %d backup params; backup = %s", len(muon), len(backup),
                [n for n, _ in backup])
    return muon, backup


def _check_named_pairs(named_params, which: str):
    for item in named_params:
        if (isinstance(item, (tuple, list)) and len(item) == 2 and isinstance(item[0], str)
                and isinstance(item[1], torch.Tensor)):
            continue
        raise TypeError(
            "validate_split expects the {} list to contain (name, param) pairs, got {!r}. Pass named parameters "
            "(e.g. model.named_parameters() or the lists from split_params_for_muon), or build the optimizer via "
            "GefenMuonHybrid.from_model(model, ...)".format(which, type(item)))


def validate_split(muon_named_params, backup_named_params, model: nn.Module = None):
    """params.py:127-187: (name, param) pairs only; no parameter twice or in
    both lists; unique names; with a model, every trainable parameter
    covered.  Returns the two lists."""
    muon_named_params = list(muon_named_params)
    backup_named_params = list(backup_named_params)
    _check_named_pairs(muon_named_params, "muon")
    _check_named_pairs(backup_named_params, "backup")
    muon_ids = {id(p) for _, p in muon_named_params}
    backup_ids = {id(p) for _, p in backup_named_params}
    if len(muon_ids) != len(muon_named_params):
        raise ValueError("Duplicate parameter object in the muon list")
    if len(backup_ids) != len(backup_named_params):
        raise ValueError("Duplicate parameter object in the backup list")
    overlap = muon_ids & backup_ids
    if overlap:
        dupes = [n for n, p in muon_named_params if id(p) in overlap]
        raise ValueError("Parameter(s) {} appear in BOTH the muon and backup lists; they would be stepped twice per "
                         "optimizer step".format(dupes))
    names = [str(n).lower() for n, _ in muon_named_params] + [str(n).lower() for n, _ in backup_named_params]
    if len(set(names)) != len(names):
        seen, dupes = set(), set()
        for n in names:
            (dupes if n in seen else seen).add(n)
        raise ValueError("Duplicate parameter name(s) {} across the muon/backup lists; the per-parameter codebook "
                         "cache keys on the name, so duplicates collide".format(sorted(dupes)))
    if model is not None:
        covered = muon_ids | backup_ids
        missing = [name for name, p in model.named_parameters() if p.requires_grad and id(p) not in covered]
        if missing:
            raise ValueError("Trainable parameter(s) {} are in neither the muon nor backup list; they would never "
                             "be optimized".format(missing))
    return muon_named_params, backup_named_params
