"""Growth and retention policy of the per-device scratch buffer
(``kairyu_amd._native.WorkspacePool``), with host tensors standing in for
device memory."""

from __future__ import annotations

import torch

from kairyu_amd._native import WorkspacePool


def _pool(minimum=16):
    state = {"capturing": False, "syncs": 0, "allocs": []}

    def allocate(index, nbytes):
        state["allocs"].append(nbytes)
        return torch.empty(nbytes, dtype=torch.uint8)

    def synchronize(index):
        state["syncs"] += 1

    return WorkspacePool(allocate, lambda index: state["capturing"], synchronize, minimum), state


def test_growth_is_geometric():
    pool, state = _pool()
    for need in range(1, 5000, 7):   # ever larger calls
        assert pool.get(0, need).numel() >= need
    # 16 -> 32 -> ... -> 8192: one allocation per doubling, not one per call
    assert state["allocs"] == [16 * 2 ** i for i in range(10)]
    assert state["syncs"] == len(state["allocs"]) - 1
    assert pool.retained == []           # nothing was captured: all released
    assert WorkspacePool.grown_size(100, 1000, 16) == 1000
    assert WorkspacePool.grown_size(100, 150, 16) == 200


def test_buffers_used_by_a_captured_graph_are_retained_and_bounded():
    pool, state = _pool()
    first = pool.get(0, 10)
    state["capturing"] = True
    assert pool.get(0, 10) is first       # handed to a graph
    state["capturing"] = False
    second = pool.get(0, 100)             # outgrows the captured buffer
    assert pool.retained == [first]
    assert state["syncs"] == 0            # never synchronizes a buffer a graph may use
    third = pool.get(0, 1000)             # `second` was never captured: released
    assert pool.retained == [first]
    assert state["syncs"] == 1
    assert sum(t.numel() for t in pool.retained) < third.numel()
    assert second.numel() == 100


def test_devices_are_independent():
    pool, _ = _pool()
    a, b = pool.get(0, 64), pool.get(1, 128)
    assert a is not b and pool.get(0, 1) is a and pool.get(1, 1) is b
