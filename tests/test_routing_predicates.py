"""Routing predicates of the fused wrapper module, as the reference's
tests/test_update_v2_dispatch.py checks them: the GEFEN_UPDATE_V2 override
forces both dispatchers; without it `_should_use_v2` follows the
SM-normalised occupancy rule and `_should_use_v2_full` its own shape table
(kernels/automatic_gefen_fused.py:23-50, 162-199).  On the CPU the CU count
is seeded into the module's per-device cache (256, an MI355X's CU count), so
the rule is evaluated without a device.  Both answers reach the same MI355X
kernels; the predicates are kept for callers that consult them.
"""
import importlib
import os

import pytest
import torch

DEV = torch.device("cuda", 0)
CUS = 256


def _reload(value):
    if value is None:
        os.environ.pop("GEFEN_UPDATE_V2", None)
    else:
        os.environ["GEFEN_UPDATE_V2"] = value
    import gefen.kernels.automatic_gefen_fused as m
    m = importlib.reload(m)
    m._SM_COUNT_BY_DEVICE[0] = CUS
    return m


@pytest.fixture
def restore_env():
    old = os.environ.get("GEFEN_UPDATE_V2")
    yield
    _reload(old)


@pytest.mark.parametrize("forced,expect", [("1", True), ("0", False), ("true", True), ("off", False),
                                           ("no", False), ("yes", True)])
def test_env_override_forces_both_dispatchers(forced, expect, restore_env):
    m = _reload(forced)
    for nb, period in ((100_000, 512), (4, 1_048_576), (4096, 1), (1, 3)):
        assert m._should_use_v2(nb, period, DEV) is expect
        assert m._should_use_v2_full(nb, period, DEV) is expect


def test_legacy_occupancy_rule(restore_env):
    m = _reload(None)
    plo, bps = m._V2_PERIOD_MAX, m._V2_BLOCKS_PER_SM
    assert m._should_use_v2(bps * CUS * 8, plo * 4, DEV) is False       # well occupied -> v1
    assert m._should_use_v2(bps * CUS * 8, plo, DEV) is True            # small period -> v2
    assert m._should_use_v2(10_000_000, 1, DEV) is True
    assert m._should_use_v2(bps * CUS - 1, 100_000, DEV) is True        # few blocks -> v2
    assert m._should_use_v2(bps * CUS, plo + 1, DEV) is False           # at the threshold -> v1
    assert m._should_use_v2(4, 512, torch.device("cpu")) is False       # non-device params never route v2


@pytest.mark.parametrize("nb,period,expect", [
    (4096, 1, False), (1_000_000, 1, True), (8192, 12, False), (262_144, 16, False),
    (1_048_576, 16, True), (4, 512, False), (512, 8192, True),
    (8193, 15, True),   # past the tiny-block bound, the legacy rule decides (period <= 16)
    (4, 4000, True),    # above the v1 period range: few blocks -> v2
])
def test_full_shape_rule(nb, period, expect, restore_env):
    m = _reload(None)
    assert m._should_use_v2_full(nb, period, DEV) is expect


def test_constants_match_the_reference(restore_env):
    m = _reload(None)
    assert (m._V2_PERIOD_MAX, m._V2_BLOCKS_PER_SM, m._CAPT_V1_FULL_TINY_NUMEL) == (16, 2, 1 << 14)
    assert (m._FULL_V1_PERIOD_MIN, m._FULL_V1_PERIOD_MAX, m._FULL_V1_TINY_NUM_BLOCKS) == (16, 2048, 1 << 13)
    assert (m._FULL_V2_LARGE_PERIOD_MIN, m._FULL_V2_PERIOD16_NUMEL) == (1 << 13, 1 << 24)
