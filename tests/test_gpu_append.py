"""KV-cache append (append_kv / append_kv_fp8) against the oracle's restatement.

The pools after the op must equal oracle.append_kv bit for bit: a copy for fp16 / bf16
pools, and for fp8 pools the bytes of oracle.quantize_e4m3 (itself pinned against torch's
float8_e4m3fn cast on every 16-bit input, tests/test_oracle_fp8.py).  Cases cover
positions at both ends of a page, rows that must be skipped (no tokens, a position past
the table, a page id outside the pool), every fp16 bit pattern through the fp8 encoder,
decoding after the append, and the *_append ops, which fuse the append into the decode and
must give bit for bit the pools and output of append_kv followed by the op.
"""
import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu

F16, BF16, F8 = torch.float16, torch.bfloat16, torch.float8_e4m3fn


def _pools(pages, hkv, ps, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    k = torch.randn(pages, hkv, ps, 128, generator=gen)
    v = torch.randn(pages, hkv, ps, 128, generator=gen)
    if dtype == F8:
        return (k / 0.05).clamp(-448, 448).to(F8), (v / 0.05).clamp(-448, 448).to(F8)
    return k.to(dtype), v.to(dtype)


# rows: (seq_len, block-table row); the pool has 12 pages
ROWS = [
    (1, [3, 0, 0]),        # first slot of the first page
    (16, [5, 7, 0]),       # last slot of page 0 (page size 16)
    (17, [1, 2, 0]),       # first slot of the second page
    (40, [9, 10, 11]),     # last page of the table
    (0, [4, 4, 4]),        # no tokens: skipped
    (49, [6, 6, 6]),       # position 48 is past the 3-column table: skipped
    (20, [8, -1, 0]),      # page id -1: skipped
    (33, [0, 2, 12]),      # page id 12 is outside the pool: skipped
]


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_append_matches_oracle(ext, gpu, dtype):
    ps, hkv, pages = 16, 4, 12
    k, v = _pools(pages, hkv, ps, dtype, seed=1)
    table = torch.tensor([r for _, r in ROWS], dtype=torch.int32)
    lens = torch.tensor([n for n, _ in ROWS], dtype=torch.int32)
    gen = torch.Generator().manual_seed(2)
    kn = torch.randn(len(ROWS), hkv, 128, generator=gen).to(dtype)
    vn = torch.randn(len(ROWS), hkv, 128, generator=gen).to(dtype)
    kg, vg = k.to(gpu), v.to(gpu)
    ext.append_kv(kn.to(gpu), vn.to(gpu), kg, vg, table.to(gpu), lens.to(gpu))
    torch.cuda.synchronize()
    k_ref, v_ref = oracle.append_kv(k, v, table, lens, kn, vn)
    assert torch.equal(kg.cpu(), k_ref) and torch.equal(vg.cpu(), v_ref)
    assert not torch.equal(k_ref, k)  # something was written


@pytest.mark.parametrize("in_dtype", [F16, BF16])
@pytest.mark.parametrize("ks,vs", [(0.05, 0.02), (1.0, 1.0 / 448)])
def test_append_fp8_matches_oracle(ext, gpu, in_dtype, ks, vs):
    ps, hkv, pages = 16, 4, 12
    k8, v8 = _pools(pages, hkv, ps, F8, seed=3)
    table = torch.tensor([r for _, r in ROWS], dtype=torch.int32)
    lens = torch.tensor([n for n, _ in ROWS], dtype=torch.int32)
    gen = torch.Generator().manual_seed(4)
    kn = (torch.randn(len(ROWS), hkv, 128, generator=gen) * 8).to(in_dtype)
    vn = (torch.randn(len(ROWS), hkv, 128, generator=gen) * 8).to(in_dtype)
    kn[0, 0, :4] = torch.tensor([0.0, -0.0, 1e4, -1e4]).to(in_dtype)  # signed zeros, saturation
    kg, vg = k8.to(gpu), v8.to(gpu)
    ext.append_kv_fp8(kn.to(gpu), vn.to(gpu), kg, vg, table.to(gpu), lens.to(gpu), ks, vs)
    torch.cuda.synchronize()
    kq = torch.from_numpy(oracle.quantize_e4m3(kn.float().numpy(), ks)).view(F8)
    vq = torch.from_numpy(oracle.quantize_e4m3(vn.float().numpy(), vs)).view(F8)
    k_ref, v_ref = oracle.append_kv(k8, v8, table, lens, kq, vq)
    assert torch.equal(kg.cpu().view(torch.uint8), k_ref.view(torch.uint8))
    assert torch.equal(vg.cpu().view(torch.uint8), v_ref.view(torch.uint8))


@pytest.mark.parametrize("scale", [1.0, 1.0 / 64])
def test_append_fp8_every_fp16_code(ext, gpu, scale):
    """All 65536 fp16 bit patterns (NaNs, infinities, subnormals, ties) through the
    kernel's e4m3 encoder: 64 rows x 8 KV heads x 128 dims, each row to its own page."""
    rows, hkv, ps = 64, 8, 16
    codes = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(F16)
    kn = codes.view(rows, hkv, 128)
    vn = codes.flip(0).view(rows, hkv, 128)
    k8 = torch.zeros(rows, hkv, ps, 128, dtype=torch.uint8).view(F8)
    v8 = torch.zeros_like(k8)
    table = torch.arange(rows, dtype=torch.int32).view(rows, 1)
    lens = torch.full((rows,), 5, dtype=torch.int32)  # slot 4 of each row's page
    kg, vg = k8.to(gpu), v8.to(gpu)
    ext.append_kv_fp8(kn.to(gpu), vn.to(gpu), kg, vg, table.to(gpu), lens.to(gpu), scale, scale)
    torch.cuda.synchronize()
    got_k = kg.cpu().view(torch.uint8)[:, :, 4].reshape(-1).numpy()
    got_v = vg.cpu().view(torch.uint8)[:, :, 4].reshape(-1).numpy()
    want_k = oracle.quantize_e4m3(kn.float().reshape(-1).numpy(), scale)
    want_v = oracle.quantize_e4m3(vn.float().reshape(-1).numpy(), scale)
    assert (got_k == want_k).all() and (got_v == want_v).all()
    assert int(kg.cpu().view(torch.uint8)[:, :, :4].abs().sum()) == 0  # other slots untouched


@pytest.mark.parametrize("dtype,ps", [(F16, 16), (BF16, 32), (F16, 5)])
def test_decode_after_append(ext, gpu, dtype, ps):
    """Append one token to each row, then the masked op attends to the grown rows."""
    lengths = [300, 17, 64, 1]
    case = make_case([n + 1 for n in lengths], 32, 8, ps, dtype, seed=ps)
    gen = torch.Generator().manual_seed(9)
    kn = torch.randn(len(lengths), 8, 128, generator=gen).to(dtype)
    vn = torch.randn(len(lengths), 8, 128, generator=gen).to(dtype)
    k, v = case.k_pages.to(gpu), case.v_pages.to(gpu)
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    ext.append_kv(kn.to(gpu), vn.to(gpu), k, v, bt, sl)
    out = torch.full((len(lengths), 32, 128), float("nan"), dtype=dtype, device=gpu)
    ws = torch.empty(len(lengths) * 32 * 2 * 130, dtype=torch.float32, device=gpu)
    bucket = max(case.seq_lens.tolist())
    ext.paged_attention_masked(case.q.to(gpu), k, v, bt, sl, out, ws, bucket, ps, 2)
    torch.cuda.synchronize()
    k_ref, v_ref = oracle.append_kv(case.k_pages, case.v_pages, case.block_table, case.seq_lens,
                                    kn, vn)
    assert torch.equal(k.cpu(), k_ref)
    ref = oracle.paged_decode(case.q, k_ref, v_ref, case.block_table, case.seq_lens)
    assert_parity(out, ref)


def test_append_validation(ext, gpu):
    k, v = _pools(4, 2, 16, F16, seed=0)
    k, v = k.to(gpu), v.to(gpu)
    kn = torch.zeros(1, 2, 128, dtype=F16, device=gpu)
    bt = torch.zeros(1, 2, dtype=torch.int32, device=gpu)
    sl = torch.ones(1, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="wrong dtype"):
        ext.append_kv(kn.to(BF16), kn.to(BF16), k, v, bt, sl)
    with pytest.raises(RuntimeError, match="Hkv mismatch"):
        ext.append_kv(torch.zeros(1, 3, 128, dtype=F16, device=gpu),
                      torch.zeros(1, 3, 128, dtype=F16, device=gpu), k, v, bt, sl)
    with pytest.raises(RuntimeError, match="batch size mismatch"):
        ext.append_kv(kn, kn, k, v, bt, torch.ones(2, dtype=torch.int32, device=gpu))
    k8, v8 = _pools(4, 2, 16, F8, seed=0)
    with pytest.raises(RuntimeError, match="k_scale"):
        ext.append_kv_fp8(kn, kn, k8.to(gpu), v8.to(gpu), bt, sl, 0.0, 1.0)
    with pytest.raises(RuntimeError, match="wrong dtype"):
        ext.append_kv_fp8(kn, kn, k, v, bt, sl, 1.0, 1.0)


@pytest.mark.parametrize("fused", [False, True])
def test_append_then_decode_in_a_hip_graph(ext, gpu, fused):
    """append_kv + the masked op (or the fused paged_attention_indexed_append) captured in
    one HIP graph and replayed several times, with eager work (pool reset, output clear)
    between replays: every replay gives the eager result."""
    lengths = [700, 33, 129]
    case = make_case(lengths, 32, 8, 16, F16, seed=21)
    gen = torch.Generator().manual_seed(22)
    kn = torch.randn(3, 8, 128, generator=gen).to(F16).to(gpu)
    vn = torch.randn(3, 8, 128, generator=gen).to(F16).to(gpu)
    k0, v0 = case.k_pages.to(gpu), case.v_pages.to(gpu)
    k, v = k0.clone(), v0.clone()
    q, bt, sl = case.q.to(gpu), case.block_table.to(gpu), case.seq_lens.to(gpu)
    out = torch.zeros(3, 32, 128, dtype=F16, device=gpu)
    ws = torch.empty(3 * 32 * 4 * 130, dtype=torch.float32, device=gpu)

    idx = torch.arange(3, dtype=torch.int32, device=gpu)

    def step():
        if fused:
            ext.paged_attention_indexed_append(q, k, v, bt, sl, idx, idx, out, ws, max(lengths),
                                               16, 4, kn, vn)
        else:
            ext.append_kv(kn, vn, k, v, bt, sl)
            ext.paged_attention_masked(q, k, v, bt, sl, out, ws, max(lengths), 16, 4)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.synchronize()
    eager_out, eager_k = out.clone(), k.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            step()
    torch.cuda.synchronize()
    for _ in range(4):
        k.copy_(k0)
        v.copy_(v0)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out) and torch.equal(k, eager_k)


def _new_tokens(b, hkv, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    return (torch.randn(b, hkv, 128, generator=gen).to(dtype),
            torch.randn(b, hkv, 128, generator=gen).to(dtype))


# (lengths, Hq, Hkv, page_size, splits, dtype); lengths count the appended token
FUSED_INDEXED = [
    ([300, 17, 64, 1], 32, 8, 16, 3, F16),
    ([700, 33, 1], 32, 4, 32, 2, BF16),        # G = 8, page 32
    ([1000, 65], 32, 1, 16, 4, BF16),          # G = 32 (two head blocks)
    ([2048], 32, 8, 16, 1, F16),               # direct launch, split inside
    ([129, 0, 96], 32, 8, 16, 2, F16),         # a row with no tokens: no append, zeros
    ([90, 41], 32, 8, 5, 2, F16),              # page 5: append kernel, then the decode
    ([31, 32, 33, 48, 49, 64], 8, 8, 16, 1, F16),  # the token at both ends of tiles and blocks
]


@pytest.mark.parametrize("lengths,hq,hkv,ps,splits,dtype", FUSED_INDEXED)
def test_fused_append_indexed_equals_append_then_decode(ext, gpu, lengths, hq, hkv, ps, splits,
                                                        dtype):
    """paged_attention_indexed_append (and paged_attention_masked_append) give bit for bit
    the output and the pools of append_kv followed by paged_attention_indexed, and match
    the oracle."""
    b = len(lengths)
    case = make_case(lengths, hq, hkv, ps, dtype, seed=sum(lengths) + ps, q_rows=b + 1)
    kn, vn = _new_tokens(b, hkv, dtype, seed=len(lengths))
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    qi = torch.arange(b, dtype=torch.int32, device=gpu).flip(0)
    oi = torch.arange(b, dtype=torch.int32, device=gpu)
    bucket = max(max(lengths), 32 * splits)
    ws = torch.empty(max(1, b * hq * splits * 130), dtype=torch.float32, device=gpu)
    q = case.q.to(gpu)

    k1, v1 = case.k_pages.to(gpu), case.v_pages.to(gpu)
    out1 = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.append_kv(kn.to(gpu), vn.to(gpu), k1, v1, bt, sl)
    ext.paged_attention_indexed(q, k1, v1, bt, sl, qi, oi, out1, ws, bucket, ps, splits)
    k2, v2 = case.k_pages.to(gpu), case.v_pages.to(gpu)
    out2 = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.paged_attention_indexed_append(q, k2, v2, bt, sl, qi, oi, out2, ws, bucket, ps, splits,
                                       kn.to(gpu), vn.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(k2, k1) and torch.equal(v2, v1)
    assert torch.equal(out2, out1)
    k_ref, v_ref = oracle.append_kv(case.k_pages, case.v_pages, case.block_table, case.seq_lens,
                                    kn, vn)
    ref = oracle.paged_decode(case.q, k_ref, v_ref, case.block_table, case.seq_lens,
                              qi.cpu(), oi.cpu())
    assert_parity(out2, ref)
    # The masked op with the append: query row b, output row b.
    k3, v3 = case.k_pages.to(gpu), case.v_pages.to(gpu)
    out3 = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    qm = q.index_select(0, qi.long()).contiguous()
    ext.paged_attention_masked_append(qm, k3, v3, bt, sl, out3, ws, bucket, ps, splits,
                                      kn.to(gpu), vn.to(gpu))
    torch.cuda.synchronize()
    assert torch.equal(k3, k1) and torch.equal(v3, v1)
    assert torch.equal(out3, out1)


@pytest.mark.parametrize("fused_merge", [False, True])
@pytest.mark.parametrize("lengths,hkv,dtype,ps", [([40, 700, 1500, 33], 8, F16, 16),
                                                  ([3000, 65, 900], 1, BF16, 16),
                                                  ([500, 2100, 64, 97], 4, BF16, 32),
                                                  ([300, 41], 8, F16, 8)])  # page 8: two launches
def test_fused_append_workqueue_equals_append_then_decode(ext, gpu, lengths, hkv, dtype, ps,
                                                          fused_merge):
    hq = 32
    case = make_case(lengths, hq, hkv, ps, dtype, seed=len(lengths) + hkv)
    meta = pkv_native.build_workqueue(lengths, list(range(len(lengths))), case.page_lists, ps, 6,
                                      False, hkv)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    bt, sl, wi, so, qi, oi = (t(meta[k]) for k in ("block_table", "seq_lens", "work_items",
                                                   "split_offsets", "q_indices", "out_indices"))
    kn, vn = _new_tokens(len(lengths), hkv, dtype, seed=7)
    slots = meta["total_partial_slots"]
    q = case.q.to(gpu)
    results = []
    for fused_append in (False, True):
        k, v = case.k_pages.to(gpu), case.v_pages.to(gpu)
        out = torch.full((len(lengths), hq, 128), float("nan"), dtype=dtype, device=gpu)
        ws = torch.empty(slots * hq * 130, dtype=torch.float32, device=gpu)
        counters = torch.zeros(len(lengths), hkv, dtype=torch.int32, device=gpu)
        args = (q, k, v, bt, sl, wi, so, counters, qi, oi, out, ws, meta["bucket_length"], ps,
                slots, fused_merge)
        if fused_append:
            ext.paged_attention_workqueue_append(*args, kn.to(gpu), vn.to(gpu))
        else:
            ext.append_kv(kn.to(gpu), vn.to(gpu), k, v, bt, sl)
            ext.paged_attention_workqueue(*args)
        torch.cuda.synchronize()
        results.append((out.cpu(), k.cpu(), v.cpu()))
    (o1, k1, v1), (o2, k2, v2) = results
    assert torch.equal(k2, k1) and torch.equal(v2, v1)
    assert torch.equal(o2, o1)
    k_ref, v_ref = oracle.append_kv(case.k_pages, case.v_pages, case.block_table, case.seq_lens,
                                    kn, vn)
    assert torch.equal(k2, k_ref) and torch.equal(v2, v_ref)
    ref = oracle.paged_decode(case.q, k_ref, v_ref, meta["block_table"], meta["seq_lens"],
                              meta["q_indices"], meta["out_indices"])
    assert_parity(o2, ref)


# rows: (seq_len, block-table row) over a 16-page pool, the skip cases of ROWS arranged so
# that no row reads a page another row appends to (the fused ops' precondition: a row's
# tail slot is read by no other row of the step)
FUSED_ROWS = [
    (1, [3, 13, 13]),      # first slot of the first page
    (16, [5, 7, 14]),      # last slot of page 0
    (17, [1, 2, 15]),      # first slot of the second page
    (40, [9, 10, 11]),     # last page of the table
    (0, [4, 4, 4]),        # no tokens: skipped
    (49, [6, 6, 6]),       # position 48 is past the 3-column table: skipped
    (20, [8, -1, 0]),      # page id -1: skipped (the decode clamps it to page 0)
    (33, [0, 12, 16]),     # page id 16 is outside the pool: skipped (decoded as page 15)
]


@pytest.mark.parametrize("op", ["indexed", "masked", "workqueue"])
def test_fused_append_skipped_rows_equal_append_then_decode(ext, gpu, op):
    """The fused append on the rows the append kernel skips (no tokens, a position past
    the 3-column table, a page id of -1, a page id outside the pool) next to ordinary
    rows: pools and output equal append_kv followed by the op, bit for bit (the decode
    clamps those lengths and page ids the same way in both)."""
    ps, hkv, hq, pages, dtype = 16, 4, 16, 16, F16
    table = torch.tensor([r for _, r in FUSED_ROWS], dtype=torch.int32)
    lens = [n for n, _ in FUSED_ROWS]
    b = len(FUSED_ROWS)
    k0, v0 = _pools(pages, hkv, ps, dtype, seed=5)
    kn, vn = (t.to(gpu) for t in _new_tokens(b, hkv, dtype, seed=6))
    gen = torch.Generator().manual_seed(7)
    q = torch.randn(b, hq, 128, generator=gen).to(dtype).to(gpu)
    bt, sl = table.to(gpu), torch.tensor(lens, dtype=torch.int32, device=gpu)
    idx = torch.arange(b, dtype=torch.int32, device=gpu)
    if op == "workqueue":
        meta = pkv_native.build_workqueue(lens, list(range(b)), [r for _, r in FUSED_ROWS], ps,
                                          2, False, hkv)
        t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
        slots = meta["total_partial_slots"]
        wi, so = t(meta["work_items"]), t(meta["split_offsets"])
        ws = torch.empty(slots * hq * 130, dtype=torch.float32, device=gpu)
    else:
        ws = torch.empty(b * hq * 2 * 130, dtype=torch.float32, device=gpu)
    results = []
    for fused in (False, True):
        k, v = k0.to(gpu), v0.to(gpu)
        out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
        if op == "workqueue":
            counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
            args = (q, k, v, bt, sl, wi, so, counters, idx, idx, out, ws, max(lens), ps, slots,
                    False)
            call = ext.paged_attention_workqueue_append if fused else ext.paged_attention_workqueue
        elif op == "indexed":
            args = (q, k, v, bt, sl, idx, idx, out, ws, 48, ps, 2)  # 3 columns of 16 tokens
            call = ext.paged_attention_indexed_append if fused else ext.paged_attention_indexed
        else:
            args = (q, k, v, bt, sl, out, ws, 48, ps, 2)
            call = ext.paged_attention_masked_append if fused else ext.paged_attention_masked
        if fused:
            call(*args, kn, vn)
        else:
            ext.append_kv(kn, vn, k, v, bt, sl)
            call(*args)
        torch.cuda.synchronize()
        results.append((out.cpu(), k.cpu(), v.cpu()))
    (o1, k1, v1), (o2, k2, v2) = results
    assert torch.equal(k2, k1) and torch.equal(v2, v1)
    assert torch.equal(o2, o1)
    k_ref, v_ref = oracle.append_kv(k0, v0, table, torch.tensor(lens, dtype=torch.int32),
                                    kn.cpu(), vn.cpu())
    assert torch.equal(k2, k_ref) and torch.equal(v2, v_ref)


@pytest.mark.parametrize("op", ["indexed", "workqueue", "indexed_fp8"])
def test_fused_append_rejected_before_any_write(ext, gpu, op):
    """A fused-append op whose workspace is too small raises before the append runs: the
    pools stay bit-identical (page 5 and fp8 pools run the append kernel inside the op)."""
    lengths, hq, hkv = [90, 41], 32, 8
    ps = 5 if op == "indexed" else 16
    case = make_case(lengths, hq, hkv, ps, F16, seed=3)
    b = len(lengths)
    kn, vn = (t.to(gpu) for t in _new_tokens(b, hkv, F16, seed=4))
    q, bt, sl = case.q.to(gpu), case.block_table.to(gpu), case.seq_lens.to(gpu)
    idx = torch.arange(b, dtype=torch.int32, device=gpu)
    out = torch.zeros(b, hq, 128, dtype=F16, device=gpu)
    small = torch.empty(16, dtype=torch.float32, device=gpu)
    if op == "indexed_fp8":
        k = (case.k_pages.float() / 0.05).clamp(-448, 448).to(F8).to(gpu)
        v = (case.v_pages.float() / 0.05).clamp(-448, 448).to(F8).to(gpu)
    else:
        k, v = case.k_pages.to(gpu), case.v_pages.to(gpu)
    k_before, v_before = k.clone(), v.clone()
    with pytest.raises(RuntimeError, match="workspace"):
        if op == "indexed":
            ext.paged_attention_indexed_append(q, k, v, bt, sl, idx, idx, out, small, 90, ps, 2,
                                               kn, vn)
        elif op == "indexed_fp8":
            ext.paged_attention_indexed_fp8_append(q, k, v, bt, sl, idx, idx, out, small, 90, ps,
                                                   2, 0.05, 0.05, kn, vn)
        else:
            meta = pkv_native.build_workqueue(lengths, list(range(b)), case.page_lists, ps, 2,
                                              False, hkv)
            t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
            counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
            ext.paged_attention_workqueue_append(
                q, k, v, t(meta["block_table"]), t(meta["seq_lens"]), t(meta["work_items"]),
                t(meta["split_offsets"]), counters, t(meta["q_indices"]), t(meta["out_indices"]),
                out, small, meta["bucket_length"], ps, meta["total_partial_slots"], False, kn, vn)
    torch.cuda.synchronize()
    view = (lambda x: x.view(torch.uint8)) if op == "indexed_fp8" else (lambda x: x)
    assert torch.equal(view(k), view(k_before)) and torch.equal(view(v), view(v_before))


def test_fused_append_validation(ext, gpu):
    case = make_case([64], 32, 8, 16, F16)
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    idx = torch.zeros(1, dtype=torch.int32, device=gpu)
    out = torch.empty(1, 32, 128, dtype=F16, device=gpu)
    ws = torch.empty(0, dtype=torch.float32, device=gpu)
    kn = torch.zeros(1, 8, 128, dtype=F16, device=gpu)
    with pytest.raises(RuntimeError, match=r"k_new must have shape"):
        ext.paged_attention_indexed_append(q, k, v, bt, sl, idx, idx, out, ws, 64, 16, 1,
                                           kn[:, :4].contiguous(), kn[:, :4].contiguous())
    with pytest.raises(RuntimeError, match="wrong dtype"):
        ext.paged_attention_indexed_append(q, k, v, bt, sl, idx, idx, out, ws, 64, 16, 1,
                                           kn.to(BF16), kn.to(BF16))


@pytest.mark.parametrize("op", ["indexed", "workqueue"])
@pytest.mark.parametrize("dtype,hkv", [(F16, 8), (BF16, 4), (F16, 1)])  # G = 4, 8, 32
def test_fused_append_fp8_equals_append_then_decode(ext, gpu, op, dtype, hkv):
    """The fp8-K/V ops with the append fused in store the e4m3 bytes of append_kv_fp8 and
    give the output of append_kv_fp8 followed by the fp8 op, bit for bit (G = 32 takes the
    separate append kernel inside the op)."""
    lengths, hq, ps, ks, vs = [700, 33, 1, 129], 32, 16, 0.05, 0.03
    b = len(lengths)
    case = make_case(lengths, hq, hkv, ps, F16, seed=hkv + 40)
    k8 = (case.k_pages.float() / ks).clamp(-448, 448).to(F8)
    v8 = (case.v_pages.float() / vs).clamp(-448, 448).to(F8)
    q = case.q.to(dtype).to(gpu)
    kn, vn = (t.to(gpu) for t in _new_tokens(b, hkv, dtype, seed=hkv))
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    results = []
    for fused in (False, True):
        k, v = k8.to(gpu), v8.to(gpu)
        out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
        if op == "indexed":
            idx = torch.arange(b, dtype=torch.int32, device=gpu)
            ws = torch.empty(b * hq * 3 * 130, dtype=torch.float32, device=gpu)
            args = (q, k, v, bt, sl, idx, idx, out, ws, max(lengths), ps, 3, ks, vs)
            if fused:
                ext.paged_attention_indexed_fp8_append(*args, kn, vn)
            else:
                ext.append_kv_fp8(kn, vn, k, v, bt, sl, ks, vs)
                ext.paged_attention_indexed_fp8(*args)
        else:
            meta = pkv_native.build_workqueue(lengths, list(range(b)), case.page_lists, ps, 5,
                                              False, hkv)
            t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
            slots = meta["total_partial_slots"]
            ws = torch.empty(slots * hq * 130, dtype=torch.float32, device=gpu)
            counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
            args = (q, k, v, t(meta["block_table"]), t(meta["seq_lens"]), t(meta["work_items"]),
                    t(meta["split_offsets"]), counters, t(meta["q_indices"]),
                    t(meta["out_indices"]), out, ws, meta["bucket_length"], ps, slots, False, ks, vs)
            if fused:
                ext.paged_attention_workqueue_fp8_append(*args, kn, vn)
            else:
                ext.append_kv_fp8(kn, vn, k, v, t(meta["block_table"]), t(meta["seq_lens"]), ks, vs)
                ext.paged_attention_workqueue_fp8(*args)
        torch.cuda.synchronize()
        results.append((out.cpu(), k.cpu().view(torch.uint8), v.cpu().view(torch.uint8)))
    (o1, k1, v1), (o2, k2, v2) = results
    assert torch.equal(k2, k1) and torch.equal(v2, v1)
    assert not torch.equal(k2, k8.view(torch.uint8))  # the append wrote
    assert torch.equal(o2, o1)
