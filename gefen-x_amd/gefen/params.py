"""Routing of parameters between Muon and the Gefen backup, and checks of a
hand-made split (reference params.py:30-187).

Rule: a trainable parameter goes to Muon when it is 2D, is not the weight of
an embedding module (identity test, so a head tied to an embedding follows
it) and its lower-cased name contains none of the backup substrings;
everything else -- embeddings, LM / classifier heads, norms, biases, other
shapes -- goes to the backup optimizer.
"""
from __future__ import annotations

import collections
import logging
from typing import Iterable, List, Sequence, Tuple

import torch
import torch.nn as nn

logger = logging.getLogger(__name__)

NamedParams = List[Tuple[str, nn.Parameter]]

# Name substrings (case-insensitive) that keep a 2D weight off Muon
# (params.py:30-37).  A routing table of the reference, kept identical.
DEFAULT_BACKUP_SUBSTRINGS: Tuple[str, ...] = (
    "embed",
    "wte",
    "wpe",
    "lm_head",
    "classifier",
    "score",
)


def is_muon_param(name: str, param, backup_substrings=DEFAULT_BACKUP_SUBSTRINGS) -> bool:
    """params.py:40-45: 2D, and no backup substring in the lower-cased name."""
    lowered = name.lower()
    return param.ndim == 2 and all(s.lower() not in lowered for s in backup_substrings)


def _embedding_param_ids(model: nn.Module) -> set:
    """Identities of the weights of every nn.Embedding / nn.EmbeddingBag
    (params.py:48-62); a tied head shares one of these objects."""
    kinds = (nn.Embedding, nn.EmbeddingBag)
    return {id(m.weight) for m in model.modules() if isinstance(m, kinds) and getattr(m, "weight", None) is not None}


def split_params_for_muon(
    model: nn.Module,
    backup_substrings: Iterable[str] = DEFAULT_BACKUP_SUBSTRINGS,
) -> Tuple[NamedParams, NamedParams]:
    """(muon, backup) lists of (name, param) pairs over the model's trainable
    parameters, in model order (params.py:65-101); logs the split."""
    subs = tuple(backup_substrings)
    embedding_ids = _embedding_param_ids(model)

    def to_muon(name, p):
        return id(p) not in embedding_ids and is_muon_param(name, p, subs)

    trainable = [(n, p) for n, p in model.named_parameters() if p.requires_grad]
    muon = [(n, p) for n, p in trainable if to_muon(n, p)]
    backup = [(n, p) for n, p in trainable if not to_muon(n, p)]
    logger.info("split_params_for_muon: Muon gets %d tensors, the backup %d: %s", len(muon), len(backup),
                [n for n, _ in backup])
    return muon, backup


def _is_named_pair(item) -> bool:
    return (isinstance(item, (tuple, list)) and len(item) == 2 and isinstance(item[0], str)
            and isinstance(item[1], torch.Tensor))


def _require_named_pairs(items: Sequence, side: str) -> None:
    """TypeError for anything but (str, tensor) pairs (params.py:104-124): a
    bare 2-row tensor would otherwise unpack into two rows."""
    bad = [item for item in items if not _is_named_pair(item)]
    if bad:
        raise TypeError(
            "validate_split: every entry of the {} list must be a (name, parameter) pair; found {!r}. Use "
            "model.named_parameters(), the lists split_params_for_muon returns, or "
            "GefenMuonHybrid.from_model(model, ...)".format(side, type(bad[0])))


def validate_split(muon_named_params, backup_named_params, model: nn.Module = None):
    """params.py:127-187: raise on a split that would step a parameter twice
    or never.  TypeError for entries that are not (name, param) pairs;
    ValueError for a parameter object listed twice on one side, listed on
    both sides, two entries whose names collide case-insensitively (the
    codebook cache keys on names), and -- given `model` -- a trainable
    parameter on neither side.  Returns the two lists."""
    lists = {"muon": list(muon_named_params), "backup": list(backup_named_params)}
    for side, items in lists.items():
        _require_named_pairs(items, side)
    owners = collections.defaultdict(list)  # id(param) -> [(side, name), ...]
    for side, items in lists.items():
        for name, p in items:
            owners[id(p)].append((side, name))
    for side in lists:
        if any(sum(1 for s, _ in entries if s == side) > 1 for entries in owners.values()):
            raise ValueError("Duplicate parameter object in the {} list".format(side))
    in_both = [name for entries in owners.values() for s, name in entries
               if s == "muon" and len({x for x, _ in entries}) == 2]
    if in_both:
        raise ValueError("Parameter(s) {} appear in BOTH the muon and backup lists, so every step would update "
                         "them twice".format(in_both))
    name_counts = collections.Counter(str(n).lower() for items in lists.values() for n, _ in items)
    clashes = sorted(n for n, c in name_counts.items() if c > 1)
    if clashes:
        raise ValueError("Duplicate parameter name(s) {} across the two lists; names key the per-parameter "
                         "codebook cache and must be unique".format(clashes))
    if model is not None:
        uncovered = [n for n, p in model.named_parameters() if p.requires_grad and id(p) not in owners]
        if uncovered:
            raise ValueError("Trainable parameter(s) {} are in neither the muon nor the backup list and would "
                             "never be updated".format(uncovered))
    return lists["muon"], lists["backup"]
