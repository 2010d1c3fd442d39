"""Parity of the four ops (HIP engine) with the repack + fp32 SDPA oracle.

Tolerances: max-abs 2e-3 (north star) and mean-abs 3e-4 (tests/smoke_test.cu:106) in
fp16 and bf16.  Case shapes follow the reference's smoke cases (tests/smoke_test.cu:
486-493) and extend them to every G in [1, 32], bf16, generic page sizes, ragged and
empty rows, indexed Q/O rows and the compact work queue.
"""
import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu

F16, BF16 = torch.float16, torch.bfloat16


def _dev(case, dev):
    return (case.q.to(dev), case.k_pages.to(dev), case.v_pages.to(dev), case.block_table.to(dev),
            case.seq_lens.to(dev))


def _ws(batch, hq, splits, dev, direct=None):
    """Workspace of a split launch; for splits == 1, ``direct = (ext, hkv, context)`` sizes
    it for the op's full internal split (empty otherwise: the single launch)."""
    if splits > 1:
        floats = max(1, batch * hq * splits * 130)
    elif direct is not None:
        ext, hkv, ctx = direct
        floats = ext.direct_workspace_floats(batch, hq, hkv, ctx)
    else:
        floats = 0
    return torch.empty(floats, dtype=torch.float32, device=dev)


# (B, Hq, Hkv, context, page_size, splits, dtype, table)
PAGED = [
    (1, 32, 8, 2048, 16, 1, F16, "random"),      # config c1 shape
    (1, 4, 1, 257, 16, 1, F16, "contiguous"),    # smoke cases (:486-493)
    (1, 8, 2, 257, 16, 4, F16, "reversed"),
    (1, 32, 8, 512, 16, 4, F16, "random"),
    (2, 32, 8, 259, 32, 3, F16, "reversed"),
    (1, 32, 4, 511, 16, 4, F16, "random"),       # G = 8
    (1, 8, 8, 256, 16, 2, F16, "random"),        # G = 1
    (1, 32, 2, 700, 16, 5, F16, "random"),       # G = 16
    (1, 32, 1, 1000, 32, 8, BF16, "random"),     # G = 32, bf16
    (3, 12, 4, 123, 8, 2, F16, "random"),        # G = 3, page 8 (generic pager)
    (2, 8, 2, 77, 5, 1, F16, "random"),          # page 5 (generic pager)
    (1, 16, 16, 64, 64, 2, BF16, "random"),
    (2, 24, 8, 100, 16, 1, BF16, "random"),
    (1, 32, 8, 8192, 16, 1, F16, "canonical"),   # canonical fragmented table
    (1, 32, 8, 8192, 16, 16, F16, "canonical"),
    (1, 32, 1, 3000, 16, 1, F16, "random"),      # G = 32 direct, split inside
    (2, 48, 2, 600, 16, 3, BF16, "reversed"),    # G = 24
    (2, 40, 2, 333, 8, 1, F16, "random"),        # G = 20, page 8 (generic pager)
    (1, 27, 1, 300, 16, 2, F16, "random"),       # G = 27
    (2, 32, 8, 3000, 256, 4, F16, "random"),     # page 256
    (1, 32, 2, 131072, 16, 64, BF16, "random"),  # 128k-token row, G = 16
    (2, 64, 8, 1500, 16, 3, F16, "reversed"),    # Hq = 64, G = 8
    (1, 64, 2, 900, 32, 1, BF16, "random"),      # Hq = 64, G = 32, direct
]


@pytest.mark.parametrize("b,hq,hkv,ctx,ps,splits,dtype,table", PAGED)
def test_paged_attention(ext, gpu, b, hq, hkv, ctx, ps, splits, dtype, table):
    case = make_case([ctx] * b, hq, hkv, ps, dtype, seed=ctx + splits, table=table)
    q, k, v, bt, _ = _dev(case, gpu)
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.paged_attention(q, k, v, bt, out, _ws(b, hq, splits, gpu, (ext, hkv, ctx)), ctx, ps, splits)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(out, ref)


# (lengths, Hq, Hkv, page_size, splits, dtype)
MASKED = [
    ([1, 31, 33, 500], 32, 8, 16, 1, F16),
    ([1, 31, 33, 500], 32, 8, 16, 4, F16),
    ([1, 31, 33, 500], 32, 8, 16, 16, BF16),
    ([5, 700, 64, 129, 1024], 8, 8, 16, 8, F16),
    ([300, 17], 32, 4, 8, 3, F16),
    ([0, 45, 96], 32, 8, 16, 2, F16),            # empty row -> zeros
    ([1024, 7000, 333], 32, 1, 32, 12, BF16),
    ([1 + (37 * i * i + 11 * i) % 600 for i in range(256)], 32, 8, 16, 2, F16),  # 256 rows
]


@pytest.mark.parametrize("lengths,hq,hkv,ps,splits,dtype", MASKED)
def test_paged_attention_masked(ext, gpu, lengths, hq, hkv, ps, splits, dtype):
    case = make_case(lengths, hq, hkv, ps, dtype, seed=sum(lengths) + splits)
    q, k, v, bt, sl = _dev(case, gpu)
    b, bucket = len(lengths), max(max(lengths), 32 * splits)
    if bt.shape[1] * ps < bucket:  # table must cover the bucket context
        bt = torch.cat([bt, bt[:, -1:].expand(b, -(-bucket // ps) - bt.shape[1])], 1).contiguous()
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.paged_attention_masked(q, k, v, bt, sl, out, _ws(b, hq, splits, gpu), bucket, ps, splits)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(out, ref)


@pytest.mark.parametrize("splits,dtype", [(1, F16), (6, F16), (3, BF16)])
def test_paged_attention_indexed(ext, gpu, splits, dtype):
    lengths = [400, 33, 1200]
    case = make_case(lengths, 32, 8, 16, dtype, seed=splits, q_rows=5)
    q, k, v, bt, sl = _dev(case, gpu)
    q_idx = torch.tensor([4, 0, 2], dtype=torch.int32)
    o_idx = torch.tensor([3, 0, 5], dtype=torch.int32)
    out = torch.full((6, 32, 128), 7.0, dtype=dtype, device=gpu)  # rows 1, 2, 4 untouched
    ext.paged_attention_indexed(q, k, v, bt, sl, q_idx.to(gpu), o_idx.to(gpu), out,
                                _ws(3, 32, splits, gpu), max(lengths), 16, splits)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens,
                              q_idx, o_idx, 6)
    assert_parity(out, ref)
    assert torch.all(out[[1, 2, 4]].float().cpu() == 7.0)


def _queue(case, requested, auto, hkv, policy=pkv_native.POLICY_REFERENCE, request_ids=None):
    ids = request_ids or list(range(len(case.seq_lens)))
    return pkv_native.build_workqueue(case.seq_lens.tolist(), ids, case.page_lists, case.page_size,
                                      requested, auto, hkv, policy)


def _run_queue(ext, gpu, case, meta, hq, hkv, fused, out_rows=None, ws_fill=None):
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    b = len(meta["seq_lens"])
    out = torch.full((out_rows or b, hq, 128), float("nan"), dtype=case.q.dtype, device=gpu)
    ws = torch.empty(meta["total_partial_slots"] * hq * 130, dtype=torch.float32, device=gpu)
    if ws_fill is not None:
        ws.fill_(ws_fill)
    counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
    ext.paged_attention_workqueue(
        case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu), t(meta["block_table"]),
        t(meta["seq_lens"]), t(meta["work_items"]), t(meta["split_offsets"]), counters,
        t(meta["q_indices"]), t(meta["out_indices"]), out, ws, meta["bucket_length"],
        case.page_size, meta["total_partial_slots"], fused)
    torch.cuda.synchronize()
    return out, counters


# (B, Hq, Hkv, N, splits, dtype): contiguous K/V [B, Hkv, N, 128]
CONTIGUOUS = [
    (1, 32, 8, 2048, 1, F16),      # direct; few units, so split inside
    (2, 32, 8, 1000, 4, F16),
    (3, 8, 8, 77, 1, BF16),        # G = 1; N not a multiple of 16
    (1, 32, 1, 3001, 8, BF16),     # G = 32
    (2, 27, 1, 500, 3, F16),       # G = 27
    (1, 4, 1, 5, 1, F16),          # N shorter than one 16-token block
    (16, 32, 8, 600, 1, F16),      # 128 units: one launch, no split
]


@pytest.mark.parametrize("b,hq,hkv,n,splits,dtype", CONTIGUOUS)
def test_attention_contiguous_and_query_head_baseline(ext, gpu, b, hq, hkv, n, splits, dtype):
    gen = torch.Generator().manual_seed(n * 3 + splits)
    q = torch.randn(b, hq, 128, generator=gen).to(dtype)
    k = torch.randn(b, hkv, n, 128, generator=gen).to(dtype)
    v = torch.randn(b, hkv, n, 128, generator=gen).to(dtype)
    ref = torch.stack([oracle.sdpa_row(q[i], k[i], v[i]) for i in range(b)])
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.attention_contiguous(qd, kd, vd, out, _ws(b, hq, splits, gpu, (ext, hkv, n)), splits)
    base = torch.full_like(out, float("nan"))
    ext.attention_query_head_baseline(qd, kd, vd, base)
    torch.cuda.synchronize()
    assert_parity(out, ref)
    assert_parity(base, ref)


# (lengths, Hq, Hkv, page_size, requested splits, auto, dtype)
QUEUE = [
    ([300, 17000, 700, 256], 32, 8, 16, 20, False, F16),   # c4-like; empty splits on short rows
    ([300, 17000, 700, 256], 32, 8, 16, 1, True, F16),     # reference auto policy
    ([64, 33, 1], 32, 8, 16, 20, False, F16),              # more splits than tiles everywhere
    ([700, 0, 300], 32, 8, 16, 6, False, F16),             # a row with no tokens (no work items)
    ([5000, 120], 32, 32, 16, 8, False, F16),              # G = 1
    ([2000, 4000, 900], 32, 1, 32, 12, False, BF16),       # G = 32 (MQA), page 32
    ([1500, 77], 32, 4, 32, 6, False, BF16),               # G = 8
    ([999, 1001], 20, 4, 8, 5, False, F16),                # G = 5, page 8
    ([3000, 40, 1200], 48, 2, 16, 7, False, F16),          # G = 24
    ([700, 2100], 27, 1, 16, 4, False, BF16),              # G = 27
]


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("lengths,hq,hkv,ps,req,auto,dtype", QUEUE)
def test_paged_attention_workqueue(ext, gpu, lengths, hq, hkv, ps, req, auto, dtype, fused):
    case = make_case(lengths, hq, hkv, ps, dtype, seed=len(lengths) * 7 + req, q_rows=len(lengths) + 2)
    ids = [len(lengths) + 1 - i for i in range(len(lengths))]  # q rows in reverse order
    meta = _queue(case, req, auto, hkv, request_ids=ids)
    out, counters = _run_queue(ext, gpu, case, meta, hq, hkv, fused)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    assert_parity(out, ref)
    assert int(counters.abs().sum()) == 0  # the fused merge leaves the counters at zero


@pytest.mark.parametrize("lengths,req", [([64, 33, 1], 20), ([300, 17000, 700, 256], 20)])
def test_workqueue_empty_split_slots_ignore_workspace_contents(ext, gpu, lengths, req):
    """Slots of splits the builder leaves empty are never written; the merge skips them
    whatever they hold (here NaN and infinities), in the max, the sum and the output."""
    case = make_case(lengths, 32, 8, 16, F16, seed=77)
    meta = _queue(case, req, False, 8)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    for fill in (float("nan"), float("inf"), -float("inf")):
        out, _ = _run_queue(ext, gpu, case, meta, 32, 8, False, ws_fill=fill)
        assert_parity(out, ref)


def _with_row_splits(case, meta, row_splits, hkv):
    """Work items and split_offsets for per-row split counts (the builder's emission
    order: row, then split, then kv head; empty splits counted in split_offsets)."""
    items, offsets = [], [0]
    for r, (length, splits) in enumerate(zip(meta["seq_lens"], row_splits)):
        tiles = -(-int(length) // 32)
        for s in range(splits):
            tb, te = tiles * s // splits, tiles * (s + 1) // splits
            if te > tb:
                items += [[r, k, s, tb, te] for k in range(hkv)]
        offsets.append(offsets[-1] + splits)
    return dict(meta, work_items=items, split_offsets=offsets, total_partial_slots=offsets[-1])


# (lengths, per-row split counts): the merge guesses a row's slot range as
# [row * S, row * S + S) when every row could have S = total_slots / batch slots.
ROW_SPLITS = [
    ([900, 1500], [3, 1]),               # total divisible by the batch, guess wrong
    ([700, 300, 2500], [2, 2, 5]),       # divisible, wrong for every row
    ([1200, 800], [4, 4]),               # uniform: guess right
    ([3000, 2000], [40, 40]),            # uniform, more than one 32-slot chunk
    ([3000, 1600], [40, 24]),            # divisible (32 per row), wrong, 40 > 32
    ([1100, 1000], [33, 31]),            # divisible, wrong by one slot
    ([500, 60, 90], [1, 1, 1]),          # one slot per row
    ([400, 2000, 30], [2, 7, 1]),        # total not divisible: no guess
]


@pytest.mark.parametrize("lengths,row_splits", ROW_SPLITS)
def test_workqueue_per_row_split_counts(ext, gpu, lengths, row_splits):
    """Merges of rows whose split counts differ, including totals that make the merge's
    fixed-split guess of the slot range look possible but wrong.  Page 8 keeps both calls
    on the per-item schedule (the balanced one needs pages of a multiple of 16), so that
    the per-item merge kernel and the fused merge fold the same states."""
    case = make_case(lengths, 32, 8, 8, F16, seed=sum(row_splits), q_rows=len(lengths) + 1)
    ids = [len(lengths) - i for i in range(len(lengths))]
    meta = _with_row_splits(case, _queue(case, 1, False, 8, request_ids=ids), row_splits, 8)
    floats = meta["total_partial_slots"] * 32 * 130
    assert ext.workqueue_schedule(len(lengths), 32, 8, 8, floats, False) == 0
    unfused, _ = _run_queue(ext, gpu, case, meta, 32, 8, False)
    fused, counters = _run_queue(ext, gpu, case, meta, 32, 8, True)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    assert_parity(unfused, ref)
    assert torch.equal(unfused, fused)  # same states, same fold order in both merges
    assert int(counters.abs().sum()) == 0


def test_workqueue_mi355x_policy(ext, gpu):
    lengths = [300, 17000, 700, 256, 31000, 900, 512, 640]
    case = make_case(lengths, 32, 8, 16, F16, seed=99)
    meta = _queue(case, 1, True, 8, policy=pkv_native.POLICY_MI355X)
    out, _ = _run_queue(ext, gpu, case, meta, 32, 8, False)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    assert_parity(out, ref)


def test_workqueue_stages_equal_combined(ext, gpu):
    """The reference's two stages (workqueue_decode, workqueue_merge: one workgroup per item,
    the reference's partial-state layout) equal the combined op with the fused merge (the
    same schedule) bit for bit, and the combined op without it bit for bit when it runs
    the per-item schedule, to fp32 rounding when it runs the balanced one."""
    lengths = [3000, 200, 9000]
    case = make_case(lengths, 32, 8, 16, F16, seed=5)
    meta = _queue(case, 20, False, 8)
    combined, _ = _run_queue(ext, gpu, case, meta, 32, 8, False)
    per_item, _ = _run_queue(ext, gpu, case, meta, 32, 8, True)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    staged = torch.full_like(combined, float("nan"))
    ws = torch.empty(meta["total_partial_slots"] * 32 * 130, dtype=torch.float32, device=gpu)
    ext.workqueue_decode(case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu),
                         t(meta["block_table"]), t(meta["seq_lens"]), t(meta["work_items"]),
                         t(meta["split_offsets"]), t(meta["q_indices"]), ws, meta["bucket_length"],
                         16, meta["total_partial_slots"])
    ext.workqueue_merge(t(meta["seq_lens"]), t(meta["split_offsets"]), t(meta["out_indices"]),
                        staged, ws, meta["total_partial_slots"])
    torch.cuda.synchronize()
    assert torch.equal(staged, per_item)
    if ext.workqueue_schedule(len(lengths), 32, 8, 16, ws.numel(), False) == 0:
        assert torch.equal(staged, combined)
    else:
        assert (staged.float() - combined.float()).abs().max().item() < 1e-3


def test_workqueue_matches_indexed_split_grid(ext, gpu):
    """Fixed S splits per row give the same tile ranges in both routes (empty slots are
    neutral in one route and skipped in the other).  A unit may be streamed by one wave
    in one route and by a whole workgroup in the other (short-unit packing depends on its
    neighbours), so the outputs agree to fp32 rounding rather than bit for bit."""
    lengths = [100, 2500, 40]
    splits = 9
    case = make_case(lengths, 32, 8, 16, F16, seed=11)
    meta = _queue(case, splits, False, 8)
    queue_out, _ = _run_queue(ext, gpu, case, meta, 32, 8, False)
    q, k, v, bt, sl = _dev(case, gpu)
    idx = torch.arange(3, dtype=torch.int32, device=gpu)
    grid_out = torch.full_like(queue_out, float("nan"))
    ext.paged_attention_indexed(q, k, v, bt, sl, idx, idx, grid_out, _ws(3, 32, splits, gpu),
                                max(lengths), 16, splits)
    torch.cuda.synchronize()
    assert (queue_out.float() - grid_out.float()).abs().max().item() < 1e-3
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(grid_out, ref)


# (op, lengths, Hq, Hkv, splits, dtype): split launches of fewer units than 3/4 of the CUs
SUBDIVIDED = [
    ("paged", [8192], 32, 8, 16, F16),         # B1 G4 8k, S 16: 128 units, 2 sub-splits
    ("paged", [3000], 8, 8, 4, BF16),          # 32 units, 8 sub-splits
    ("masked", [3000, 100], 32, 8, 8, F16),    # short row: empty sub-splits
    ("indexed", [2500, 33, 900], 32, 8, 4, BF16),
    ("contiguous", [8192], 32, 8, 16, F16),    # the reference's B1 G4 8k performance case
]


def _split_op(ext, gpu, op, case, lengths, hq, hkv, splits, floats):
    """One launch of ``op`` with a workspace of ``floats`` fp32 elements."""
    q, k, v, bt, sl = _dev(case, gpu)
    b, ctx = len(lengths), max(lengths)
    ws = torch.empty(floats, dtype=torch.float32, device=gpu)
    out = torch.full((b, hq, 128), float("nan"), dtype=case.q.dtype, device=gpu)
    if op == "paged":
        ext.paged_attention(q, k, v, bt, out, ws, ctx, 16, splits)
    elif op == "masked":
        ext.paged_attention_masked(q, k, v, bt, sl, out, ws, ctx, 16, splits)
    elif op == "indexed":
        idx = torch.arange(b, dtype=torch.int32, device=gpu).flip(0).contiguous()
        ext.paged_attention_indexed(q, k, v, bt, sl, idx, idx, out, ws, ctx, 16, splits)
    else:  # the row's pages laid end to end: [1, Hkv, ctx, 128]
        pages = case.block_table[0, :-(-ctx // 16)].long()
        kc, vc = (p[pages].permute(1, 0, 2, 3).reshape(1, hkv, -1, 128)[:, :, :ctx].contiguous()
                  for p in (case.k_pages, case.v_pages))
        ext.attention_contiguous(q, kc.to(gpu), vc.to(gpu), out, ws, splits)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("op,lengths,hq,hkv,splits,dtype", SUBDIVIDED)
def test_split_launch_subdivided(ext, gpu, op, lengths, hq, hkv, splits, dtype):
    """With the workspace of split_workspace_floats the op cuts each split into sub-splits
    (merged together); it matches the oracle, and the reference-sized workspace (caller's
    split only) and an in-between size give the same output to fp32 rounding."""
    case = make_case(lengths, hq, hkv, 16, dtype, seed=len(lengths) * 7 + splits)
    b, ctx = len(lengths), max(lengths)
    ref_floats = b * hq * splits * 130
    full = ext.split_workspace_floats(b, hq, hkv, ctx, splits)
    assert full >= 2 * ref_floats  # the launch is sub-split
    if op == "indexed":
        idx = torch.arange(b, dtype=torch.int32).flip(0)
        ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                                  case.seq_lens, idx, idx, b)
    else:
        ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    outs = [_split_op(ext, gpu, op, case, lengths, hq, hkv, splits, f)
            for f in (full, ref_floats + (full - ref_floats) // 2, ref_floats)]
    for out in outs:
        assert_parity(out, ref)
    for out in outs[1:]:
        assert (out.float() - outs[0].float()).abs().max().item() < 1e-3


def test_split_partial_states_match_oracle(ext, gpu):
    """The workspace holds the reference's partial-state format (cuh:615-632): per
    (row, head, split) m in natural-log units of the scaled score, l, acc[128]."""
    b, hq, hkv, ctx, splits = 2, 8, 2, 700, 5
    case = make_case([ctx] * b, hq, hkv, 16, F16, seed=3)
    q, k, v, bt, _ = _dev(case, gpu)
    ws = _ws(b, hq, splits, gpu)
    out = torch.empty(b, hq, 128, dtype=F16, device=gpu)
    ext.paged_attention(q, k, v, bt, out, ws, ctx, 16, splits)
    torch.cuda.synchronize()
    n = b * hq * splits
    w = ws.cpu()
    m, l, acc = w[:n].view(b, hq, splits), w[n:2 * n].view(b, hq, splits), w[2 * n:].view(b, hq, splits, 128)
    ranges = oracle.split_bounds(-(-ctx // 32), splits)
    for row in range(b):
        kk, vv = oracle.gather_row(case.k_pages, case.v_pages, case.block_table[row], ctx)
        rm, rl, racc = oracle.split_partials(case.q[row], kk, vv, ranges)
        assert torch.allclose(m[row].double(), torch.from_numpy(rm), atol=1e-4, rtol=1e-4)
        # l and acc are relative to each split's own max; compare after normalising.
        assert torch.allclose(l[row].double(), torch.from_numpy(rl), rtol=2e-3, atol=1e-3)
        assert torch.allclose(acc[row].double() / l[row].double()[..., None],
                              torch.from_numpy(racc / rl[..., None]), atol=2e-3)


def test_deterministic_and_page_relocation_invariant(ext, gpu):
    """Moving every page to another physical slot (and updating the table) reads the same
    logical tokens in the same order, so the output is bit-identical."""
    lengths = [1500, 40, 777]
    case = make_case(lengths, 32, 8, 16, F16, seed=21, extra_pages=40)
    meta = _queue(case, 20, False, 8)
    a, _ = _run_queue(ext, gpu, case, meta, 32, 8, False)
    b, _ = _run_queue(ext, gpu, case, meta, 32, 8, False)
    assert torch.equal(a, b)
    perm = torch.randperm(case.k_pages.shape[0], generator=torch.Generator().manual_seed(1))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(len(perm))
    moved = make_case(lengths, 32, 8, 16, F16, seed=21, extra_pages=40)
    moved.k_pages = case.k_pages[inv]  # physical slot p now holds old page inv[p]
    moved.v_pages = case.v_pages[inv]
    moved.page_lists = [[int(perm[p]) for p in row] for row in case.page_lists]
    moved.q = case.q
    meta2 = _queue(moved, 20, False, 8)
    c, _ = _run_queue(ext, gpu, moved, meta2, 32, 8, False)
    assert torch.equal(a, c)


def test_split_count_invariance(ext, gpu):
    ctx = 4096
    case = make_case([ctx], 32, 8, 16, F16, seed=8)
    q, k, v, bt, _ = _dev(case, gpu)
    outs = []
    for s in (1, 2, 7, 32, 128):
        out = torch.empty(1, 32, 128, dtype=F16, device=gpu)
        ext.paged_attention(q, k, v, bt, out, _ws(1, 32, s, gpu), ctx, 16, s)
        outs.append(out.float())
    torch.cuda.synchronize()
    for o in outs[1:]:
        assert (o - outs[0]).abs().max().item() < 1e-3


def test_hip_graph_replay(ext, gpu):
    lengths = [2000, 300, 5000, 64]
    case = make_case(lengths, 32, 8, 16, F16, seed=13)
    meta = _queue(case, 20, False, 8)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    args = [case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu), t(meta["block_table"]),
            t(meta["seq_lens"]), t(meta["work_items"]), t(meta["split_offsets"]),
            torch.zeros(4, 8, dtype=torch.int32, device=gpu), t(meta["q_indices"]),
            t(meta["out_indices"])]
    out = torch.zeros(4, 32, 128, dtype=F16, device=gpu)
    ws = torch.empty(meta["total_partial_slots"] * 32 * 130, dtype=torch.float32, device=gpu)
    tail = [meta["bucket_length"], 16, meta["total_partial_slots"], False]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # eager run on the capture stream
        ext.paged_attention_workqueue(*args, out, ws, *tail)
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            ext.paged_attention_workqueue(*args, out, ws, *tail)
    torch.cuda.synchronize()
    for _ in range(4):
        out.zero_()
        ws.fill_(3.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_validation_errors(ext, gpu):
    case = make_case([64], 32, 8, 16, F16)
    q, k, v, bt, sl = _dev(case, gpu)
    out = torch.empty(1, 32, 128, dtype=F16, device=gpu)
    empty = torch.empty(0, dtype=torch.float32, device=gpu)
    with pytest.raises(RuntimeError, match="num_splits"):
        ext.paged_attention(q, k, v, bt, out, _ws(1, 32, 4, gpu), 64, 16, 4)  # 4 > ceil(64/32)
    with pytest.raises(RuntimeError, match="workspace"):
        ext.paged_attention(q, k, v, bt, out, empty, 64, 16, 2)
    with pytest.raises(RuntimeError, match="G=Hq/Hkv"):
        q66 = torch.zeros(1, 66, 128, dtype=F16, device=gpu)
        ext.paged_attention(q66, k[:, :2].contiguous(), v[:, :2].contiguous(), bt,
                            torch.empty(1, 66, 128, dtype=F16, device=gpu), empty, 64, 16, 1)
    with pytest.raises(RuntimeError, match="wrong dtype"):
        ext.paged_attention(q, k.to(BF16), v.to(BF16), bt, out, empty, 64, 16, 1)
    with pytest.raises(RuntimeError, match="block_table has"):
        ext.paged_attention(q, k, v, bt, out, empty, 4096, 16, 1)
    kc = torch.zeros(1, 8, 64, 128, dtype=F16, device=gpu)
    with pytest.raises(RuntimeError, match="num_splits"):
        ext.attention_contiguous(q, kc, kc, out, _ws(1, 32, 4, gpu), 4)  # 4 > ceil(64/32)
    with pytest.raises(RuntimeError, match="workspace"):
        ext.attention_contiguous(q, kc, kc, out, empty, 2)
    with pytest.raises(RuntimeError, match="v shape mismatch"):
        ext.attention_query_head_baseline(q, kc, kc[:, :, :32].contiguous(), out)


def test_misaligned_workspace_is_rejected_before_launch(ext, gpu):
    """Partial states are accessed with 16-byte vector loads and stores: a workspace that
    is not 16-byte aligned (here a float32 tensor offset by one element) is rejected on the
    host, and nothing is launched (the output keeps its sentinel)."""
    lengths = [700, 40]
    case = make_case(lengths, 32, 8, 16, F16, seed=3)
    q, k, v, bt, sl = _dev(case, gpu)
    meta = _queue(case, 4, False, 8)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    floats = max(meta["total_partial_slots"], 2 * 64) * 32 * 130
    ws = torch.empty(floats + 4, dtype=torch.float32, device=gpu)[1:]
    assert ws.data_ptr() % 16 == 4
    out = torch.full((2, 32, 128), float("nan"), dtype=F16, device=gpu)
    counters = torch.zeros(2, 8, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        ext.paged_attention_masked(q, k, v, bt, sl, out, ws, 704, 16, 4)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        ext.paged_attention(q[:1].contiguous(), k, v, bt[:1].contiguous(), out[:1], ws, 704, 16, 1)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        ext.paged_attention_workqueue(q, k, v, t(meta["block_table"]), t(meta["seq_lens"]),
                                      t(meta["work_items"]), t(meta["split_offsets"]), counters,
                                      t(meta["q_indices"]), t(meta["out_indices"]), out, ws,
                                      meta["bucket_length"], 16, meta["total_partial_slots"], False)
    with pytest.raises(RuntimeError, match="16-byte aligned"):
        ext.workqueue_merge(t(meta["seq_lens"]), t(meta["split_offsets"]), t(meta["out_indices"]),
                            out, ws, meta["total_partial_slots"])
    torch.cuda.synchronize()
    assert torch.isnan(out.float()).all()


@pytest.mark.parametrize("op", ["masked", "indexed"])
def test_lengths_and_page_ids_outside_the_table_are_clamped(ext, gpu, op):
    """Inputs the reference would read out of bounds with: a length past the table's
    capacity is clamped to max_pages * page_size, a negative length counts as 0 (zeros),
    and a page id outside the pool is clamped into it (-7 -> 0, 10**6 -> pages - 1).  The
    expected result is the oracle on the same inputs with those rules applied on the host."""
    lengths = [100, 64, 40, 77]
    case = make_case(lengths, 32, 8, 16, F16, seed=31)
    pages, cols = case.k_pages.shape[0], case.block_table.shape[1]
    bt = case.block_table.clone()
    bt[1, 1], bt[1, 2] = -7, 10 ** 6
    sl = torch.tensor([100 + 500, 64, 40, -5], dtype=torch.int32)
    bt_ref = bt.clamp(0, pages - 1)
    sl_ref = sl.clamp(0, cols * 16)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, bt_ref, sl_ref)
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    out = torch.full((4, 32, 128), float("nan"), dtype=F16, device=gpu)
    ws = _ws(4, 32, 2, gpu)
    if op == "masked":
        ext.paged_attention_masked(q, k, v, bt.to(gpu), sl.to(gpu), out, ws, cols * 16, 16, 2)
    else:
        idx = torch.arange(4, dtype=torch.int32, device=gpu)
        ext.paged_attention_indexed(q, k, v, bt.to(gpu), sl.to(gpu), idx, idx, out, ws,
                                    cols * 16, 16, 2)
    torch.cuda.synchronize()
    assert sl_ref.tolist() == [cols * 16, 64, 40, 0]
    assert_parity(out, ref)
