"""Checkpoint cross-compatibility with the reference, host side.

tests/golden/ckpt_<case>.pt are Gefen.state_dict() files written by the
reference package itself (gefen.py:4558-4707) after three CPU steps of the
bf16 trajectory cases (factored and block second moment), loaded here with
torch.load(weights_only=True).  Checks:
  * this build loads them (gefen.py:5456-5707 semantics): saved dtypes kept
    although the parameters are bf16, counters as ints, codebook, global step
    and names restored;
  * this build's state_dict of the loaded state has the reference's layout
    (top-level keys, per-parameter keys, dtypes and shapes, group keys and the
    per-group metadata), so the reference can load what this build writes;
  * the loader's refusals: a different deterministic policy, quantised momentum
    without a codebook, metadata on only some groups.
The GPU continuation of these checkpoints against the reference's own resumed
trajectory is tests/test_gpu_checkpoint_compat.py.
"""
import copy
import os

import numpy as np
import pytest
import torch

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CASES = ["fact_bf16", "block_bf16"]


def _load(case):
    sd = torch.load(os.path.join(GOLD, "ckpt_%s.pt" % case), weights_only=True)
    ref = np.load(os.path.join(GOLD, "ckpt_%s.npz" % case))
    return sd, ref


def _opt(case, ref, device="cpu", **kw):
    from gefen import Gefen
    pre = int(ref["pre"])
    params = [(n, torch.nn.Parameter(torch.from_numpy(ref["p%d_%s" % (pre, n)]).to(torch.bfloat16).to(device)))
              for n in ("w", "b")]
    opt = Gefen(params, lr=6e-5, betas=(0.9, 0.999), eps=1e-8, weight_decay=float(ref["wd"]),
                factored_v_2d=bool(ref["factored"]), **kw)
    return params, opt


def _schema(sd):
    out = {"top": sorted(sd.keys())}
    for pid, st in sd["state"].items():
        out[pid] = {k: ((tuple(v.shape), v.dtype) if torch.is_tensor(v) else type(v).__name__) for k, v in st.items()}
    out["groups"] = [sorted(g.keys()) for g in sd["param_groups"]]
    out["meta"] = [sorted(g["_gefen_checkpoint_metadata"].keys()) for g in sd["param_groups"]]
    return out


@pytest.mark.parametrize("case", CASES)
def test_reference_checkpoint_loads(case):
    sd, ref = _load(case)
    params, opt = _opt(case, ref)
    opt.load_state_dict(copy.deepcopy(sd))
    assert opt._gefen_global_step == 3
    assert torch.equal(opt._gefen_codebook.cpu(), sd["gefen_codebook"])
    for pid, (name, p) in enumerate(params):
        st, saved = opt.state[p], sd["state"][pid]
        assert st["name"] == name
        for k, v in saved.items():
            if torch.is_tensor(v):
                assert st[k].dtype == v.dtype and torch.equal(st[k], v), (name, k)
            else:
                assert st[k] == v and type(st[k]) is type(v), (name, k)


@pytest.mark.parametrize("case", CASES)
def test_state_dict_has_reference_layout(case):
    sd, ref = _load(case)
    _, opt = _opt(case, ref)
    opt.load_state_dict(copy.deepcopy(sd))
    ours = opt.state_dict()
    assert _schema(ours) == _schema(sd)
    for pid in sd["state"]:
        for k, v in sd["state"][pid].items():
            w = ours["state"][pid][k]
            assert (torch.equal(w, v) if torch.is_tensor(v) else w == v), (pid, k)
    for g_ref, g_ours in zip(sd["param_groups"], ours["param_groups"]):
        for k in ("lr", "beta1", "beta2", "eps", "weight_decay", "param_names", "param_names_synthesized", "params"):
            assert g_ours[k] == g_ref[k], k
        m_ref, m_ours = g_ref["_gefen_checkpoint_metadata"], g_ours["_gefen_checkpoint_metadata"]
        assert m_ours["format_version"] == m_ref["format_version"] and m_ours["global_step"] == m_ref["global_step"]
        assert torch.equal(m_ours["codebook"], m_ref["codebook"])
        assert m_ours["device_anchor"].dtype == torch.uint8 and m_ours["device_anchor"].numel() == 1


def test_fresh_optimizer_state_dict_names_every_parameter():
    from gefen import Gefen
    params = [("w", torch.nn.Parameter(torch.zeros(4, 8))), torch.nn.Parameter(torch.zeros(8))]
    opt = Gefen([{"params": params}], lr=1e-3)
    sd = opt.state_dict()
    assert {pid: st["name"] for pid, st in sd["state"].items()} == {0: "w", 1: "group_0_param_1"}
    assert sd["param_groups"][0]["param_names_synthesized"] == [False, True]


def test_load_refuses_mismatched_checkpoints():
    sd, ref = _load("fact_bf16")
    _, opt = _opt("fact_bf16", ref, deterministic=True)
    with pytest.raises(ValueError, match="deterministic"):
        opt.load_state_dict(copy.deepcopy(sd))
    _, opt = _opt("fact_bf16", ref)
    bad = copy.deepcopy(sd)
    bad["gefen_codebook"] = None
    for g in bad["param_groups"]:
        g["_gefen_checkpoint_metadata"]["codebook"] = None
    with pytest.raises(ValueError, match="codebook"):
        opt.load_state_dict(bad)
    bad = copy.deepcopy(sd)
    bad["gefen_global_step"] = 7
    with pytest.raises(ValueError, match="global steps disagree"):
        opt.load_state_dict(bad)


def test_loading_a_codebookless_state_clears_the_codebook():
    """gefen.py:5632-5641: the codebook is restored unconditionally, so a
    checkpoint taken before step 1 (no codebook) clears a stale one and the
    next step learns it again."""
    sd, ref = _load("fact_bf16")
    params, opt = _opt("fact_bf16", ref)
    opt.load_state_dict(copy.deepcopy(sd))
    assert opt._gefen_codebook is not None
    _, fresh = _opt("fact_bf16", ref)
    fresh_sd = fresh.state_dict()
    assert fresh_sd["gefen_codebook"] is None
    opt.load_state_dict(fresh_sd)
    assert opt._gefen_codebook is None
    assert opt._gefen_codebook_by_device == {}
    assert opt._gefen_global_step == 0


def _state_equal(a, b):
    if torch.is_tensor(b):
        return torch.is_tensor(a) and a.dtype == b.dtype and torch.equal(a, b)
    if isinstance(b, dict):
        return isinstance(a, dict) and set(a) == set(b) and all(_state_equal(a[k], b[k]) for k in b)
    if isinstance(b, (list, tuple)):
        return len(a) == len(b) and all(_state_equal(x, y) for x, y in zip(a, b))
    return a == b


def test_determinism_policy_tags():
    """tests/test_deterministic_mode.py (reference): a checkpoint of the other
    policy is refused before anything changes, also in the DCP shape (group
    metadata only); tags must be real bools at both levels; an untagged
    legacy checkpoint loads under the live policy; a matching tag loads."""
    sd, ref = _load("fact_bf16")  # written with deterministic=False
    assert sd["gefen_deterministic"] is False
    _, opt = _opt("fact_bf16", ref, deterministic=True)
    before = copy.deepcopy(opt.state_dict())
    with pytest.raises(ValueError, match="intentional state migration"):
        opt.load_state_dict(copy.deepcopy(sd))
    assert _state_equal(opt.state_dict(), before)
    dcp = {"state": copy.deepcopy(sd["state"]), "param_groups": copy.deepcopy(sd["param_groups"])}
    with pytest.raises(ValueError, match="intentional state migration"):
        opt.load_state_dict(dcp)
    assert _state_equal(opt.state_dict(), before)
    for tag in (None, 0, 1, "true"):
        bad = copy.deepcopy(sd)
        bad["gefen_deterministic"] = tag
        _, o = _opt("fact_bf16", ref)
        b0 = copy.deepcopy(o.state_dict())
        with pytest.raises(ValueError, match="top-level deterministic policy must be a bool"):
            o.load_state_dict(bad)
        assert _state_equal(o.state_dict(), b0)
    bad = copy.deepcopy(sd)
    bad["param_groups"][0]["_gefen_checkpoint_metadata"]["deterministic"] = 1
    _, o = _opt("fact_bf16", ref)
    with pytest.raises(ValueError, match="parameter-group deterministic policy must be a bool"):
        o.load_state_dict(bad)
    legacy = copy.deepcopy(sd)
    legacy.pop("gefen_deterministic")
    for g in legacy["param_groups"]:
        g["_gefen_checkpoint_metadata"].pop("deterministic")
    _, o = _opt("fact_bf16", ref, deterministic=True)
    o.load_state_dict(legacy)
    assert o._deterministic is True
    _, o = _opt("fact_bf16", ref, deterministic=False)
    o.load_state_dict(copy.deepcopy(sd))
    assert o._gefen_global_step == 3
