"""The balanced schedule of the work-queue op (equal tile shares per wave over every
(row, kv head) pair of a complete queue, then a merge of each pair's pieces) against the
repack + fp32 SDPA oracle, against the per-item schedule (same result to fp32 rounding),
through its two stages, under HIP graph replay, with the fused append and fp8 K/V; and
the rules of pkv_workqueue_schedule."""
import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16, BF16, F8 = torch.float16, torch.bfloat16, torch.float8_e4m3fn


def _meta(case, splits, hkv, ids=None):
    ids = ids or list(range(len(case.seq_lens)))
    return pkv_native.build_workqueue(case.seq_lens.tolist(), ids, case.page_lists, case.page_size,
                                      splits, False, hkv)


def _dev_meta(meta, gpu):
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    return {k: t(meta[k]) for k in ("block_table", "seq_lens", "work_items", "split_offsets",
                                    "q_indices", "out_indices")}


def _run(ext, gpu, case, meta, hkv, floats, k=None, v=None, out_rows=None, kv=None, ws_fill=None):
    """The combined op with a workspace of ``floats`` fp32 elements."""
    d = _dev_meta(meta, gpu)
    hq = case.q.shape[1]
    b = len(meta["seq_lens"])
    out = torch.full((out_rows or b, hq, 128), float("nan"), dtype=case.q.dtype, device=gpu)
    ws = torch.empty(floats, dtype=torch.float32, device=gpu)
    if ws_fill is not None:
        ws.fill_(ws_fill)
    counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
    k = case.k_pages.to(gpu) if k is None else k
    v = case.v_pages.to(gpu) if v is None else v
    args = (case.q.to(gpu), k, v, d["block_table"], d["seq_lens"], d["work_items"],
            d["split_offsets"], counters, d["q_indices"], d["out_indices"], out, ws,
            meta["bucket_length"], case.page_size, meta["total_partial_slots"], False)
    if kv is None:
        ext.paged_attention_workqueue(*args)
    else:
        ext.paged_attention_workqueue_fp8(*args, kv[0], kv[1])
    torch.cuda.synchronize()
    return out


def _balanced_floats(ext, case, meta, hkv):
    b, hq = len(meta["seq_lens"]), case.q.shape[1]
    floats = max(meta["total_partial_slots"] * hq * 130,
                 pkv_native.workqueue_balanced_workspace_bytes(b, hq, hkv) // 4)
    assert ext.workqueue_schedule(b, hq, hkv, case.page_size, floats, False) == 1
    return floats


# (lengths, Hq, Hkv, page_size, splits, dtype)
CASES = [
    ([20000, 300, 700, 1, 5000, 64, 31000, 513], 32, 8, 16, 20, F16),   # C4-like, G = 4
    ([3000, 0, 1500, 33], 32, 8, 16, 6, F16),                            # a row with no tokens
    ([9000, 2000], 8, 8, 16, 4, BF16),                                   # G = 1
    ([7000, 65, 12000], 32, 4, 32, 5, BF16),                             # G = 8, page 32
    ([4000, 600, 8100], 32, 2, 16, 3, F16),                              # G = 16
    ([31, 32, 33, 1] * 18, 32, 8, 16, 2, F16),                           # 72 rows: two row chunks
    ([40 + 13 * i for i in range(200)], 16, 8, 16, 2, F16),              # 200 rows, G = 2
    # 24 rows x 32 heads: two merge waves per (row, query head) on 256 CUs
    ([25000 if i % 8 == 0 else 200 + 97 * i for i in range(24)], 32, 8, 16, 3, BF16),
    # 72 rows x 32 heads: one merge wave, two long rows with more than 32 groups per pair
    ([30000 if i % 36 == 0 else 100 + 7 * i for i in range(72)], 32, 8, 16, 2, F16),
    # 2 rows x 2 kv heads: pairs over hundreds of waves, folded by the wide merge
    ([30000, 9000], 16, 2, 16, 5, BF16),
    # G = 1 with an odd number of pairs: (pairs + waves) x G states is odd, padded to even
    # so that the states' acc (read with 16-byte loads by the wide fold) stays aligned
    ([3000, 500, 9000], 1, 1, 16, 4, F16),
]


@pytest.mark.parametrize("lengths,hq,hkv,ps,splits,dtype", CASES)
def test_balanced_schedule_matches_oracle(ext, gpu, lengths, hq, hkv, ps, splits, dtype):
    case = make_case(lengths, hq, hkv, ps, dtype, seed=len(lengths) + hkv, q_rows=len(lengths) + 2)
    ids = [(3 * i + 1) % (len(lengths) + 2) for i in range(len(lengths))]
    meta = _meta(case, splits, hkv, ids)
    out = _run(ext, gpu, case, meta, hkv, _balanced_floats(ext, case, meta, hkv))
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    assert_parity(out, ref)
    again = _run(ext, gpu, case, meta, hkv, _balanced_floats(ext, case, meta, hkv))
    assert torch.equal(out, again)  # the schedule depends on the sizes only


@pytest.mark.parametrize("lengths,hq,hkv", [([40, 70], 32, 8), ([1, 33, 2], 32, 4), ([90], 16, 2)])
def test_balanced_few_positions_ignore_workspace_contents(ext, gpu, lengths, hq, hkv):
    """With fewer positions than waves (T < V) most waves hold none, and the groups of a
    pair's range that such waves would own are never written: the merge skips them
    whatever they hold (NaN, infinities)."""
    case = make_case(lengths, hq, hkv, 16, F16, seed=5)
    meta = _meta(case, 4, hkv, list(range(len(lengths))))
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    floats = _balanced_floats(ext, case, meta, hkv)
    assert ext.workqueue_schedule(len(lengths), hq, hkv, 16, floats, False) == 1
    for fill in (float("nan"), float("inf"), -float("inf")):
        assert_parity(_run(ext, gpu, case, meta, hkv, floats, ws_fill=fill), ref)


def test_balanced_equals_per_item_schedule(ext, gpu):
    """Same queue, two workspace sizes: the reference size (per-item schedule: two splits
    per row leave no room for the pieces) and the balanced size; fp32 rounding apart."""
    lengths, hq, hkv = [20000, 300, 700, 5000, 64, 31000, 513, 1900], 32, 8
    case = make_case(lengths, hq, hkv, 16, F16, seed=4)
    meta = _meta(case, 2, hkv)
    ref_floats = meta["total_partial_slots"] * hq * 130
    assert ext.workqueue_schedule(len(lengths), hq, hkv, 16, ref_floats, False) == 0
    per_item = _run(ext, gpu, case, meta, hkv, ref_floats)
    balanced = _run(ext, gpu, case, meta, hkv, _balanced_floats(ext, case, meta, hkv))
    assert (per_item.float() - balanced.float()).abs().max().item() < 1e-3
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    assert_parity(per_item, ref)
    assert_parity(balanced, ref)


@pytest.mark.parametrize("balanced", [False, True])
@pytest.mark.parametrize("kv_fp8", [False, True])
def test_stages_equal_combined(ext, gpu, balanced, kv_fp8):
    lengths, hq, hkv = [9000, 200, 3000, 17], 32, 8
    case = make_case(lengths, hq, hkv, 16, F16, seed=6)
    meta = _meta(case, 4, hkv)
    floats = _balanced_floats(ext, case, meta, hkv) if balanced else meta["total_partial_slots"] * hq * 130
    assert ext.workqueue_schedule(len(lengths), hq, hkv, 16, floats, False) == int(balanced)
    k, v = case.k_pages.to(gpu), case.v_pages.to(gpu)
    scales = (0.05, 0.04)
    if kv_fp8:
        k = (k.float() / scales[0]).clamp(-448, 448).to(F8)
        v = (v.float() / scales[1]).clamp(-448, 448).to(F8)
    combined = _run(ext, gpu, case, meta, hkv, floats, k, v, kv=scales if kv_fp8 else None)
    d = _dev_meta(meta, gpu)
    staged = torch.full_like(combined, float("nan"))
    ws = torch.empty(floats, dtype=torch.float32, device=gpu)
    for stage in (1, 2):
        ext.paged_attention_workqueue_stage(
            stage, case.q.to(gpu), k, v, d["block_table"], d["seq_lens"], d["work_items"],
            d["split_offsets"], d["q_indices"], d["out_indices"], staged, ws,
            meta["bucket_length"], 16, meta["total_partial_slots"], kv_fp8, *scales)
    torch.cuda.synchronize()
    assert torch.equal(staged, combined)
    kd = oracle.dequantize_e4m3(k.cpu(), scales[0]) if kv_fp8 else case.k_pages
    vd = oracle.dequantize_e4m3(v.cpu(), scales[1]) if kv_fp8 else case.v_pages
    ref = oracle.paged_decode(case.q, kd, vd, meta["block_table"], meta["seq_lens"],
                              meta["q_indices"], meta["out_indices"])
    assert_parity(combined, ref)


def test_balanced_fused_append_equals_append_then_decode(ext, gpu):
    lengths, hq, hkv = [3000, 41, 700, 1, 1500], 32, 8
    case = make_case(lengths, hq, hkv, 16, F16, seed=8)
    meta = _meta(case, 5, hkv)
    floats = _balanced_floats(ext, case, meta, hkv)
    d = _dev_meta(meta, gpu)
    gen = torch.Generator().manual_seed(9)
    kn = torch.randn(len(lengths), hkv, 128, generator=gen).half().to(gpu)
    vn = torch.randn(len(lengths), hkv, 128, generator=gen).half().to(gpu)
    results = []
    for fused in (False, True):
        k, v = case.k_pages.to(gpu), case.v_pages.to(gpu)
        out = torch.full((len(lengths), hq, 128), float("nan"), dtype=F16, device=gpu)
        ws = torch.empty(floats, dtype=torch.float32, device=gpu)
        counters = torch.zeros(len(lengths), hkv, dtype=torch.int32, device=gpu)
        args = (case.q.to(gpu), k, v, d["block_table"], d["seq_lens"], d["work_items"],
                d["split_offsets"], counters, d["q_indices"], d["out_indices"], out, ws,
                meta["bucket_length"], 16, meta["total_partial_slots"], False)
        if fused:
            ext.paged_attention_workqueue_append(*args, kn, vn)
        else:
            ext.append_kv(kn, vn, k, v, d["block_table"], d["seq_lens"])
            ext.paged_attention_workqueue(*args)
        torch.cuda.synchronize()
        results.append((out.cpu(), k.cpu(), v.cpu()))
    (o1, k1, v1), (o2, k2, v2) = results
    assert torch.equal(k2, k1) and torch.equal(v2, v1) and torch.equal(o2, o1)
    ref = oracle.paged_decode(case.q, k1, v1, meta["block_table"], meta["seq_lens"],
                              meta["q_indices"], meta["out_indices"])
    assert_parity(o2, ref)


def test_balanced_schedule_in_a_hip_graph(ext, gpu):
    lengths, hq, hkv = [12000, 300, 5000, 64], 32, 8
    case = make_case(lengths, hq, hkv, 16, F16, seed=10)
    meta = _meta(case, 20, hkv)
    floats = _balanced_floats(ext, case, meta, hkv)
    d = _dev_meta(meta, gpu)
    out = torch.zeros(len(lengths), hq, 128, dtype=F16, device=gpu)
    ws = torch.empty(floats, dtype=torch.float32, device=gpu)
    counters = torch.zeros(len(lengths), hkv, dtype=torch.int32, device=gpu)
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    call = lambda: ext.paged_attention_workqueue(
        q, k, v, d["block_table"], d["seq_lens"], d["work_items"], d["split_offsets"], counters,
        d["q_indices"], d["out_indices"], out, ws, meta["bucket_length"], 16,
        meta["total_partial_slots"], False)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.synchronize()
    call()
    torch.cuda.synchronize()
    eager = out.clone()
    for _ in range(3):
        out.zero_()
        ws.fill_(5.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_schedule_rules(ext, gpu):
    big = 1 << 26
    assert ext.workqueue_schedule(8, 32, 8, 16, big, False) == 1
    assert ext.workqueue_schedule(8, 32, 8, 16, big, True) == 0       # fused merge
    assert ext.workqueue_schedule(8, 32, 1, 16, big, False) == 0      # G = 32
    assert ext.workqueue_schedule(8, 32, 8, 8, big, False) == 0       # page 8
    assert ext.workqueue_schedule(257, 32, 8, 16, big, False) == 0    # more than 256 rows
    need = pkv_native.workqueue_balanced_workspace_bytes(8, 32, 8) // 4
    assert ext.workqueue_schedule(8, 32, 8, 16, need, False) == 1
    assert ext.workqueue_schedule(8, 32, 8, 16, need - 1, False) == 0


@pytest.mark.parametrize("balanced", [False, True])
def test_lengths_and_page_ids_outside_the_table_are_clamped(ext, gpu, balanced):
    """The work-queue op in both schedules on inputs the reference would read out of bounds
    with: a length past the table's capacity is clamped to max_pages * page_size, a negative
    length counts as 0 (zeros), a page id outside the pool is clamped into it.  Expected: the
    oracle on the same inputs with those rules applied on the host."""
    lengths, hq, hkv = [100, 64, 40, 77], 32, 8
    case = make_case(lengths, hq, hkv, 16, F16, seed=31)
    meta = _meta(case, 2, hkv)
    bt = torch.as_tensor(meta["block_table"], dtype=torch.int32)
    pages, cols = case.k_pages.shape[0], bt.shape[1]
    bt[1, 1], bt[1, 2] = -7, 10 ** 6
    sl = torch.tensor([100 + 500, 64, 40, -5], dtype=torch.int32)
    meta = dict(meta, block_table=bt.tolist(), seq_lens=sl.tolist())
    bt_ref, sl_ref = bt.clamp(0, pages - 1), sl.clamp(0, cols * 16)
    floats = (_balanced_floats(ext, case, meta, hkv) if balanced
              else meta["total_partial_slots"] * hq * 130)
    assert ext.workqueue_schedule(4, hq, hkv, 16, floats, False) == int(balanced)
    out = _run(ext, gpu, case, meta, hkv, floats)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, bt_ref, sl_ref,
                              meta["q_indices"], meta["out_indices"])
    assert sl_ref.tolist() == [cols * 16, 64, 40, 0]
    assert_parity(out, ref)
