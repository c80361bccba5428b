"""CPU: the host-side row planning of FusedHeadLoss (testt_amd/head.py: _RowPlan) and the
sequence bounds of the varlen attention (testt_amd/attention.py: cu_seqlens_of), checked against
direct constructions on small cases (no kernel runs)."""

import torch

from testt_amd import attention, head


def _plan_reference(targets, chunk):
    labelled = (targets != head.IGNORE_INDEX).tolist()
    slot, gather, counts, before, seen = [], [], [], [], 0
    n_lab = sum(labelled)
    for c in range(0, len(labelled), chunk):
        before.append(seen)
        local = 0
        for lab in labelled[c:c + chunk]:
            if lab:
                slot.append(local)
                gather.append(seen)
                local += 1
                seen += 1
            else:
                slot.append(-1)
                gather.append(n_lab)
        counts.append(local)
    return slot, gather, counts, before, n_lab


def test_row_plan_matches_direct_construction():
    g = torch.Generator().manual_seed(3)
    for rows, chunk in ((1, 4), (37, 8), (100, 7), (64, 64), (130, 50)):
        targets = torch.randint(0, 50, (rows,), generator=g)
        targets[torch.rand(rows, generator=g) < 0.35] = head.IGNORE_INDEX
        if rows > 5:
            targets[:3] = head.IGNORE_INDEX          # a chunk may start with ignored rows
        for denominator in (11, torch.tensor(11.5)):
            plan = head._RowPlan(targets, denominator, chunk)
            slot, gather, counts, before, n_lab = _plan_reference(targets, chunk)
            assert plan.slot.dtype == torch.int32 and plan.slot.tolist() == slot
            assert plan.gather.dtype == torch.int64 and plan.gather.tolist() == gather
            assert plan.counts == counts and plan.lab_before == before
            assert plan.n_labelled == n_lab
            assert plan.denominator == float(denominator)


def test_row_plan_all_ignored_and_all_labelled():
    plan = head._RowPlan(torch.full((9,), head.IGNORE_INDEX), 4.0, 4)
    assert plan.n_labelled == 0 and plan.counts == [0, 0, 0]
    assert plan.slot.tolist() == [-1] * 9 and plan.gather.tolist() == [0] * 9
    plan = head._RowPlan(torch.arange(9), 4.0, 4)
    assert plan.counts == [4, 4, 1] and plan.lab_before == [0, 4, 8]
    assert plan.slot.tolist() == [0, 1, 2, 3, 0, 1, 2, 3, 0]
    assert plan.gather.tolist() == list(range(9))


def test_grad_unit_rule():
    """_grad_unit: the power of two nearest denominator * 64, clamped to [1, 2^16]
    (solution/head.py:79-84)."""
    assert head._grad_unit(1843) == 2.0 ** 17 / 2 ** 1   # round(log2 1843) = 11 -> 2^17 -> 2^16
    assert head._grad_unit(1) == 64.0
    assert head._grad_unit(0) == 1.0
    assert head._grad_unit(100) == 2.0 ** 13


def test_cu_seqlens_of_sorted_positions():
    mask = torch.tensor([[1, 1, 1, 0, 0], [0, 0, 0, 0, 0], [1, 1, 1, 1, 1], [1, 0, 0, 0, 0]])
    pos = mask.reshape(-1).nonzero().squeeze(1)
    cu = attention.cu_seqlens_of(pos, 4, 5)
    assert cu.dtype == torch.int32 and cu.tolist() == [0, 3, 3, 8, 9]
    # cached on the tensor, rebuilt when it changes
    assert attention.cu_seqlens_of(pos, 4, 5) is cu
    pos[8] = 20                                # past the last row: not counted
    assert attention.cu_seqlens_of(pos, 4, 5).tolist() == [0, 3, 3, 8, 8]
    # positions with gaps inside a row (left padding) keep the row's bounds
    mask = torch.tensor([[0, 0, 1, 1], [0, 1, 1, 1]])
    pos = mask.reshape(-1).nonzero().squeeze(1)
    assert attention.cu_seqlens_of(pos, 2, 4).tolist() == [0, 2, 5]
