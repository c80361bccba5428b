"""CPU: the host-side launch planning of nf4.unpack_groups (the prepared launch kept on the
first weight of a list): a different grouping of the same weights, a replaced weight and a
dropped weight each get a plan of their own, and a plan keeps no weight alive.  The per-weight
kernel plans are stubbed (no device, no kernel call)."""

import gc
import weakref

import pytest
import torch

from testt_amd import nf4


class _Weight:
    """Stands in for a Params4bit: only identity and a shape matter to the group planner."""

    def __init__(self, rows, cols):
        self.rows, self.cols = rows, cols


@pytest.fixture
def stub_plans(monkeypatch):
    def plan(w, device):
        return ((1, 2, 3, 4, 5, 6), w.rows * w.cols // 2, 64, 256, ())

    monkeypatch.setattr(nf4, "_plan", plan)
    monkeypatch.setattr(nf4, "_plan_key", lambda w, device: (device, id(w)))
    monkeypatch.setattr(nf4, "weight_shape", lambda w: (w.rows, w.cols))


def _plan_for(groups, device=torch.device("cpu")):
    flat_w, offsets, stacks, total = [], [], [], 0
    for weights in groups:
        rows = [w.rows for w in weights]
        cols = weights[0].cols
        stacks.append((total, sum(rows), cols))
        r0 = 0
        for w, n in zip(weights, rows):
            flat_w.append(w)
            offsets.append(total + r0 * cols)
            r0 += n
        total += -(-sum(rows) * cols // nf4._GROUP_ALIGN) * nf4._GROUP_ALIGN
    return nf4._group_plan(groups, device, flat_w, offsets, stacks, total)


def test_regrouping_gets_its_own_stacks(stub_plans):
    a, b, c = _Weight(8, 64), _Weight(4, 64), _Weight(4, 64)
    p1 = _plan_for([[a, b], [c]])
    assert p1.stacks == [(0, 12, 64), (768, 4, 64)]
    p2 = _plan_for([[a], [b, c]])
    assert p2 is not p1 and p2.stacks == [(0, 8, 64), (512, 8, 64)]
    p3 = _plan_for([[a, b, c]])
    assert p3.stacks == [(0, 16, 64)] and p3.total == 1024
    assert _plan_for([[a, b, c]]) is p3           # the same list reuses the prepared plan


def test_replaced_or_dropped_weight_is_replanned(stub_plans):
    a, b, c = _Weight(8, 64), _Weight(4, 64), _Weight(4, 64)
    p1 = _plan_for([[a, b, c]])
    d = _Weight(4, 64)
    p2 = _plan_for([[a, b, d]])
    assert p2 is not p1 and len(p2.launches) == 1
    assert _plan_for([[a, b]]) is not p2           # fewer weights, same first weight


def test_plan_keeps_no_weight_alive(stub_plans):
    a = _Weight(8, 64)
    replaced = []
    for _ in range(3):
        b = _Weight(4, 64)
        replaced.append(weakref.ref(b))
        _plan_for([[a, b]])
        del b
    gc.collect()
    assert all(ref() is None for ref in replaced)  # no plan held a replaced weight
    first = weakref.ref(a)
    gc.disable()
    try:
        del a
        # no cycle: the first weight goes with its last reference, without a cyclic collection
        assert first() is None
    finally:
        gc.enable()
