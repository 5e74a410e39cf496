"""GPU: the hand-built rule scenarios (tests/golden/scenarios.py; the reference's
tests/hangame_rules50_test.cpp and tests/terminal50_test.cpp situations as rows) through
the HIP engine: observe, step with events, branch (every legal action of each first row
plus an illegal and an out-of-range one, with and without the children's observation),
start, hands and stock, all identical to what the reference build recorded."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.conftest import GOLDEN, announce
from tests.test_gpu_engine import assert_observe_equal, assert_step_equal, to_np

pytestmark = pytest.mark.gpu

DEV = "cuda"


def test_scenarios_match_reference_fixture(ext):
    announce("hand-built rule scenarios vs reference fixture")
    fx = np.load(GOLDEN / "scenarios.npz")

    def dev(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)

    rows = dev(fx["step_row"])
    n = rows.shape[0]
    assert_observe_equal(ext.observe(rows),
                         (fx["features"], fx["legal"], fx["player"], fx["done"], fx["status"]),
                         "scenario observation")
    out = ext.step_events_indexed(rows, torch.arange(n, device=DEV), dev(fx["step_action"]))
    assert_step_equal(out, [fx[k] for k in ("reward", "step_done", "nagari", "step_status",
                                            "committed", "events")], "scenario step")
    assert np.array_equal(to_np(rows), fx["after"])
    rows = dev(fx["step_row"])
    out = ext.step(rows, dev(fx["step_action"]))
    assert_step_equal(out, [fx[k] for k in ("reward", "step_done", "nagari", "step_status",
                                            "committed")], "scenario step (plain)")
    assert np.array_equal(to_np(rows), fx["after"])

    first = dev(fx["first"])
    ids, acts = dev(fx["branch_scenario"]), dev(fx["branch_action"])
    child = ext.branch_indexed(first, ids, acts)
    assert np.array_equal(to_np(child[0]), fx["children"])
    assert_step_equal(child[1:], [fx[k] for k in ("b_reward", "b_done", "b_nagari",
                                                  "b_status", "b_committed")], "branch")
    fused = ext.branch_observe_indexed(first, ids, acts)
    for j in range(6):
        assert torch.equal(fused[j], child[j]), j
    observed = ext.observe(child[0])
    for j in range(5):
        assert torch.equal(fused[6 + j], observed[j]), j
    assert np.array_equal(to_np(first), fx["first"])  # parents untouched
    k = torch.arange(first.shape[0], device=DEV)
    assert np.array_equal(to_np(ext.start(first)), fx["start"])
    assert np.array_equal(to_np(ext.hands_indexed(first, k)), fx["hands"])
    assert np.array_equal(to_np(ext.stock_indexed(first, k)), fx["stock"])
