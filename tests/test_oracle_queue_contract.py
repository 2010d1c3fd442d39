"""Pins oracle.attention.workqueue_decode, the work-queue op's result for any queue.

Every check compares against a formulation that does not use the oracle's per-slot
partial states and merge: fp32 SDPA over whole rows or over truncated rows
(paged_decode), or fp64 attention over an explicit list of keys.  A planted mistake (the
merge reading only the builder's non-empty splits) must fail.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oracle
from oracle import workqueue as wq
from paged_cases import make_case
import queue_cases as qc

HQ, HKV = 8, 2


def _run(case, items, offsets, total_slots=None):
    b = len(case.seq_lens)
    return oracle.workqueue_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                                   case.seq_lens, torch.tensor(items, dtype=torch.int32),
                                   offsets, list(range(b)), list(range(b)), b, total_slots)


def _truth(case, covered=None):
    lens = case.seq_lens.tolist()
    if covered is not None:
        lens = [min(n, 32 * p) for n, p in zip(lens, covered)]
    return oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                               torch.tensor(lens, dtype=torch.int32))


LENGTHS = [40, 300, 1, 700, 64]


@pytest.mark.parametrize("splits", [1, 3, 8, 40])
def test_builder_queue_is_attention_over_each_row(splits):
    case = make_case(LENGTHS, HQ, HKV, 16, torch.float32, seed=splits)
    meta = wq.build_workqueue(LENGTHS, list(range(5)), case.page_lists, 16, splits, False, HKV)
    out = _run(case, meta["work_items"], meta["split_offsets"])
    assert (out - _truth(case)).abs().max().item() < 1e-5


@pytest.mark.parametrize("splits", [2, 4, 30])
def test_explicit_empty_items_and_other_partitions(splits):
    case = make_case(LENGTHS, HQ, HKV, 16, torch.float32, seed=7)
    items, offsets, _ = qc.front_loaded(LENGTHS, HKV, splits)
    assert (_run(case, items, offsets) - _truth(case)).abs().max().item() < 1e-5
    items, offsets, _ = qc.random_partition(LENGTHS, HKV, splits, seed=splits)
    assert (_run(case, items, offsets) - _truth(case)).abs().max().item() < 1e-5


def test_prefix_queue_is_attention_over_the_prefix():
    case = make_case(LENGTHS, HQ, HKV, 16, torch.float32, seed=3)
    items, offsets, covered = qc.random_partition(LENGTHS, HKV, 5, seed=1,
                                                  prefix=lambda t: (t + 1) // 2)
    assert covered != [qc.tiles_of(n) for n in LENGTHS]
    out = _run(case, items, offsets)
    assert (out - _truth(case, covered)).abs().max().item() < 1e-5


def test_formula_markers_take_the_row_local_bounds():
    case = make_case(LENGTHS, HQ, HKV, 16, torch.float32, seed=5)
    meta = wq.build_workqueue(LENGTHS, list(range(5)), case.page_lists, 16, 6, False, HKV)
    out = _run(case, qc.formula_markers(meta["work_items"]), meta["split_offsets"])
    assert (out - _truth(case)).abs().max().item() < 1e-5


def test_overlapping_ranges_count_each_token_once_per_item():
    """Two items of one row naming the same tile: its keys enter the softmax twice."""
    case = make_case([70], 2, 1, 16, torch.float32, seed=11)
    items = [[0, 0, 0, 0, 2], [0, 0, 1, 1, 3]]  # tile 1 twice
    out = _run(case, items, [0, 2])
    k, v = oracle.gather_row(case.k_pages, case.v_pages, case.block_table[0], 70)
    keep = list(range(0, 70)) + list(range(32, 64))
    ref = oracle.attention_fp64(case.q[0], k[:, keep], v[:, keep])
    assert np.abs(out[0].numpy() - ref).max() < 1e-5


def test_unwritten_slots_and_invalid_items_are_neutral():
    case = make_case([100, 50], 2, 1, 16, torch.float32, seed=13)
    # row 0: slots 0 and 2 written, slot 1 never; bad items are ignored
    items = [[0, 0, 0, 0, 2], [0, 0, 2, 2, 4], [5, 0, 0, 0, 1], [0, 3, 0, 0, 1],
             [1, 0, 1, 0, 1], [1, 0, 0, 0, 2]]
    out = _run(case, items, [0, 3, 4])
    assert (out - _truth(case)).abs().max().item() < 1e-5


def test_planted_builder_only_merge_fails():
    """The merge rule of a builder-only engine (skip slots whose row-local bounds are
    empty) drops tiles of a caller's queue."""
    case = make_case([60], 2, 1, 16, torch.float32, seed=17)  # 2 tiles
    items, offsets, _ = qc.front_loaded([60], 1, 4)  # tiles in splits 0 and 1
    t, s = 2, 4
    live = [sp for sp in range(s) if t * sp // s < t * (sp + 1) // s]  # splits 1 and 3
    planted = [it for it in items if it[2] in live]
    good = _run(case, items, offsets)
    bad = _run(case, planted, offsets)
    assert (good - _truth(case)).abs().max().item() < 1e-5
    assert (bad - _truth(case)).abs().max().item() > 1e-2
