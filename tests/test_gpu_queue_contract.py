"""The work-queue op on caller-built queues, in each of its schedules, against the
oracle's restatement of the reference's kernels (oracle.attention.workqueue_decode).

The reference honours each item's tile range (cuh:298-337), writes the neutral state for
an item without tiles (cuh:340-363) and folds every slot of a row (cuh:753-784); its fused
merge waits for one arrival per slot (cuh:659).  Each queue below writes every slot once,
so the reference defines its result:
- (a) fewer tiles than splits, the tiles in the first splits, explicit empty items after;
- (b) other partitions of a row's tiles over its splits, in any item order;
- (c) items that cover only a prefix of each row's tiles;
- per-row split counts (rows of one slot included), and the row-local bounds given as -1.
Every schedule is forced: the balanced one (a workspace that holds it), the per-item one
(the reference's workspace size, below the balanced size here) and the fused merge.  The
builder's own queue in another item order is also run: the balanced schedule then takes
its fallback, and the merge skips the slots of the builder's empty splits.
"""
import pytest
import torch

import pkv_native
from oracle import attention as oracle
from oracle import workqueue as wq
from paged_cases import assert_parity, make_case
import queue_cases as qc

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


def _call(ext, gpu, case, items, offsets, hkv, schedule, ws_fill=float("nan"), q_idx=None):
    """The combined op: schedule "balanced", "per_item" or "fused"."""
    b, hq = len(case.seq_lens), case.q.shape[1]
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    slots = offsets[-1]
    floats = slots * hq * 130
    if schedule == "balanced":
        floats = max(floats, pkv_native.workqueue_balanced_workspace_bytes(b, hq, hkv) // 4)
    expect = 1 if schedule == "balanced" else 0
    assert ext.workqueue_schedule(b, hq, hkv, case.page_size, floats, schedule == "fused") == expect
    ws = torch.full((floats,), ws_fill, dtype=torch.float32, device=gpu)
    out = torch.full((b + 1, hq, 128), float("nan"), dtype=case.q.dtype, device=gpu)
    counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
    q_idx = list(range(b)) if q_idx is None else q_idx
    ext.paged_attention_workqueue(
        case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu), t(case.block_table),
        t(case.seq_lens), t(items), t(offsets), counters, t(q_idx), t(list(range(b))), out, ws,
        int(case.seq_lens.max()), case.page_size, slots, schedule == "fused")
    torch.cuda.synchronize()
    assert int(counters.abs().sum()) == 0
    return out[:b]


def _oracle(case, items, offsets, q_idx=None):
    b = len(case.seq_lens)
    q_idx = list(range(b)) if q_idx is None else q_idx
    return oracle.workqueue_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                                   case.seq_lens, torch.tensor(items, dtype=torch.int32), offsets,
                                   q_idx, list(range(b)), b)


SCHEDULES = ["balanced", "per_item", "fused"]
# (lengths, Hq, Hkv, splits, dtype)
SHAPES = [
    ([40, 300, 1, 700, 64, 2000], 32, 8, 4, F16),     # G = 4, short rows with T < S
    ([5000, 33, 900], 16, 2, 6, BF16),                # G = 8
    ([1200, 100], 8, 8, 3, F16),                      # G = 1
]


@pytest.mark.parametrize("schedule", SCHEDULES)
@pytest.mark.parametrize("lengths,hq,hkv,splits,dtype", SHAPES)
@pytest.mark.parametrize("queue", ["front_loaded", "random_partition", "prefix", "markers"])
def test_caller_queue_matches_reference(ext, gpu, queue, lengths, hq, hkv, splits, dtype, schedule):
    case = make_case(lengths, hq, hkv, 16, dtype, seed=len(lengths) + splits)
    if queue == "front_loaded":
        items, offsets, _ = qc.front_loaded(lengths, hkv, splits)
    elif queue == "random_partition":
        items, offsets, _ = qc.random_partition(lengths, hkv, splits, seed=splits)
    elif queue == "prefix":
        items, offsets, covered = qc.random_partition(lengths, hkv, splits, seed=3,
                                                      prefix=lambda t: (2 * t + 2) // 3)
    else:
        meta = wq.build_workqueue(lengths, list(range(len(lengths))), case.page_lists, 16,
                                  splits, False, hkv)
        items, offsets = qc.formula_markers(meta["work_items"]), meta["split_offsets"]
    print(f"queue={queue} schedule={schedule} lengths={lengths} G={hq // hkv} S={splits}", flush=True)
    out = _call(ext, gpu, case, items, offsets, hkv, schedule)
    assert_parity(out, _oracle(case, items, offsets))


@pytest.mark.parametrize("schedule", SCHEDULES)
def test_per_row_split_counts_with_single_slot_rows(ext, gpu, schedule):
    lengths = [900, 60, 3000, 200]
    case = make_case(lengths, 32, 8, 16, F16, seed=41)
    items, offsets, _ = qc.per_row_splits(lengths, 8, [3, 1, 7, 2], seed=5)
    out = _call(ext, gpu, case, items, offsets, 8, schedule)
    assert_parity(out, _oracle(case, items, offsets))


@pytest.mark.parametrize("schedule", ["balanced", "per_item"])
def test_builder_queue_in_another_order(ext, gpu, schedule):
    """The builder's items kv-head-major instead of split-major: not the builder's queue
    (the balanced schedule takes its fallback), and with empty splits (T < S) not a queue
    that writes every slot (the merge skips those slots, which hold NaN here)."""
    lengths = [40, 5000, 300, 64]
    case = make_case(lengths, 32, 8, 16, F16, seed=43)
    meta = wq.build_workqueue(lengths, list(range(4)), case.page_lists, 16, 20, False, 8)
    items = sorted(meta["work_items"], key=lambda it: (it[0], it[1], it[2]))
    assert items != meta["work_items"]
    out = _call(ext, gpu, case, items, meta["split_offsets"], 8, schedule)
    assert_parity(out, oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                                           case.seq_lens))


def test_schedules_agree_on_a_caller_queue(ext, gpu):
    """Both unfused schedules and the fused merge give one answer (to fp32 rounding and
    the output's own rounding) on a queue the reference defines."""
    lengths = [3000, 70, 1100, 20000]
    case = make_case(lengths, 32, 8, 16, F16, seed=47)
    items, offsets, _ = qc.random_partition(lengths, 8, 5, seed=9, prefix=lambda t: t - 1)
    outs = [_call(ext, gpu, case, items, offsets, 8, s).float() for s in SCHEDULES]
    ref = _oracle(case, items, offsets)
    for o in outs:
        assert_parity(o.half(), ref)
    assert (outs[0] - outs[1]).abs().max().item() < 2e-3
    assert (outs[1] - outs[2]).abs().max().item() == 0  # same states, same fold order


def test_balanced_stages_equal_combined_on_fallback(ext, gpu):
    """Stage 1 then stage 2 of the balanced schedule equal the combined call on a queue
    that takes the fallback."""
    lengths = [700, 64, 2500]
    hq, hkv = 32, 8
    case = make_case(lengths, hq, hkv, 16, F16, seed=53)
    items, offsets, _ = qc.front_loaded(lengths, hkv, 5)
    combined = _call(ext, gpu, case, items, offsets, hkv, "balanced")
    b = len(lengths)
    floats = max(offsets[-1] * hq * 130, pkv_native.workqueue_balanced_workspace_bytes(b, hq, hkv) // 4)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    ws = torch.full((floats,), float("nan"), dtype=torch.float32, device=gpu)
    staged = torch.full((b, hq, 128), float("nan"), dtype=F16, device=gpu)
    args = (case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu), t(case.block_table),
            t(case.seq_lens), t(items), t(offsets), t(list(range(b))), t(list(range(b))), staged, ws,
            int(case.seq_lens.max()), 16, offsets[-1], False, 1.0, 1.0)
    ext.paged_attention_workqueue_stage(1, *args)
    ext.paged_attention_workqueue_stage(2, *args)
    torch.cuda.synchronize()
    assert torch.equal(staged, combined)
