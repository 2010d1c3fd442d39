"""Launches of few, long units: the whole-line K path.

A direct launch (num_splits == 1) with no workspace to split into, or a split launch
whose workspace holds no sub-splits, of at most half as many units as the GPU has CUs and
at least 16 tiles (512 tokens) per unit, runs one workgroup per unit whose K loads take
whole 128-byte lines straight into LDS (the reference's own C1 call: one row, 8 KV heads,
`workspace` empty).  Each case here is such a launch, against the repack + fp32 SDPA
oracle at the parity bar (max-abs 2e-3, mean-abs 3e-4): every op with a grid launch
(paged, masked, indexed, contiguous, the query-head baseline, the fused append), direct
and split, fp16 and bf16, G from 1 to 16, page sizes that are multiples of 16, ragged and
empty rows, rows of one or two tiles in a long bucket (one wave alone), partial last
tiles and long rows.  The fused append must equal the append followed by the same decode
bit for bit, as on every other path.
"""
import pytest
import torch

from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu

F16, BF16 = torch.float16, torch.bfloat16


def _empty(gpu):
    return torch.empty(0, dtype=torch.float32, device=gpu)


# (B, Hq, Hkv, context, page_size, dtype, table)
PAGED = [
    (1, 32, 8, 2048, 16, F16, "random"),       # config c1
    (1, 32, 8, 8192, 16, F16, "canonical"),
    (4, 32, 8, 1000, 32, BF16, "random"),      # partial last tile, page 32
    (1, 8, 8, 545, 16, F16, "random"),         # G = 1, partial last tile
    (1, 32, 8, 520, 16, BF16, "reversed"),
    (2, 64, 4, 777, 64, F16, "random"),        # G = 16, page 64
    (3, 12, 4, 1023, 16, BF16, "random"),      # G = 3
    (2, 32, 8, 3000, 256, F16, "reversed"),    # page 256
    (16, 32, 8, 600, 16, F16, "random"),       # 128 units: half of 256 CUs
    (1, 16, 8, 65536, 16, BF16, "random"),     # G = 2, 64k-token row
]


@pytest.mark.parametrize("b,hq,hkv,ctx,ps,dtype,table", PAGED)
def test_paged_direct_without_workspace(ext, gpu, b, hq, hkv, ctx, ps, dtype, table):
    case = make_case([ctx] * b, hq, hkv, ps, dtype, seed=ctx + b, table=table)
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.paged_attention(case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu),
                        case.block_table.to(gpu), out, _empty(gpu), ctx, ps, 1)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(out, ref)


@pytest.mark.parametrize("lengths,hq,hkv,ps,dtype", [
    ([1, 31, 33, 500, 0, 2049], 32, 8, 16, F16),   # ragged, one empty row (zeros)
    ([64, 65, 95, 96, 97], 8, 2, 32, BF16),         # tile and page edges, G = 4
    ([4000, 1, 17], 16, 16, 16, F16),               # G = 1
])
def test_masked_direct_without_workspace(ext, gpu, lengths, hq, hkv, ps, dtype):
    case = make_case(lengths, hq, hkv, ps, dtype, seed=sum(lengths))
    b, bucket = len(lengths), max(max(lengths), 1024)
    bt = case.block_table
    if bt.shape[1] * ps < bucket:  # the table covers the bucket
        bt = torch.cat([bt, bt[:, -1:].expand(b, -(-bucket // ps) - bt.shape[1])], 1).contiguous()
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.paged_attention_masked(case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu),
                               bt.to(gpu), case.seq_lens.to(gpu), out, _empty(gpu), bucket, ps, 1)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(out, ref)


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_indexed_direct_without_workspace(ext, gpu, dtype):
    lengths = [400, 33, 1200]
    case = make_case(lengths, 32, 8, 16, dtype, seed=11, q_rows=5)
    q_idx = torch.tensor([4, 0, 2], dtype=torch.int32)
    o_idx = torch.tensor([3, 0, 5], dtype=torch.int32)
    out = torch.full((6, 32, 128), 7.0, dtype=dtype, device=gpu)  # rows 1, 2, 4 untouched
    ext.paged_attention_indexed(case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu),
                                case.block_table.to(gpu), case.seq_lens.to(gpu), q_idx.to(gpu),
                                o_idx.to(gpu), out, _empty(gpu), max(lengths), 16, 1)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens,
                              q_idx, o_idx, 6)
    assert_parity(out, ref)
    assert torch.all(out[[1, 2, 4]].float().cpu() == 7.0)


@pytest.mark.parametrize("b,hq,hkv,n,dtype", [
    (1, 32, 8, 2048, F16),
    (3, 8, 8, 577, BF16),    # G = 1, N not a multiple of 16
    (1, 4, 1, 517, F16),
    (2, 32, 4, 5000, BF16),  # G = 8
])
def test_contiguous_direct_without_workspace(ext, gpu, b, hq, hkv, n, dtype):
    gen = torch.Generator().manual_seed(n + b)
    q = torch.randn(b, hq, 128, generator=gen).to(dtype)
    k = torch.randn(b, hkv, n, 128, generator=gen).to(dtype)
    v = torch.randn(b, hkv, n, 128, generator=gen).to(dtype)
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.attention_contiguous(qd, kd, vd, out, _empty(gpu), 1)
    base = torch.full_like(out, float("nan"))  # one unit per query head: B * Hq units
    ext.attention_query_head_baseline(qd, kd, vd, base)
    torch.cuda.synchronize()
    ref = torch.stack([oracle.sdpa_row(q[i], k[i], v[i]) for i in range(b)])
    assert_parity(out, ref)
    assert_parity(base, ref)


@pytest.mark.parametrize("lengths,dtype", [([1, 40, 1000, 33, 2048], F16), ([16, 17, 511], BF16)])
def test_fused_append_direct_without_workspace(ext, gpu, lengths, dtype):
    """The fused append (new token taken in the decode) equals the append followed by the
    same decode, bit for bit, and the pools it leaves are the same; both match the oracle
    over the appended pools."""
    hq, hkv, ps = 32, 8, 16
    b = len(lengths)
    case = make_case(lengths, hq, hkv, ps, dtype, seed=sum(lengths), extra_pages=4)
    gen = torch.Generator().manual_seed(b)
    kn = torch.randn(b, hkv, 128, generator=gen).to(dtype).to(gpu)
    vn = torch.randn(b, hkv, 128, generator=gen).to(dtype).to(gpu)
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    qi = torch.arange(b, dtype=torch.int32, device=gpu)
    q = case.q.to(gpu)
    k1, v1 = case.k_pages.to(gpu), case.v_pages.to(gpu)
    out1 = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.append_kv(kn, vn, k1, v1, bt, sl)
    ext.paged_attention_indexed(q, k1, v1, bt, sl, qi, qi, out1, _empty(gpu), max(lengths), ps, 1)
    k2, v2 = case.k_pages.to(gpu), case.v_pages.to(gpu)
    out2 = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.paged_attention_indexed_append(q, k2, v2, bt, sl, qi, qi, out2, _empty(gpu), max(lengths),
                                       ps, 1, kn, vn)
    torch.cuda.synchronize()
    assert torch.equal(k2, k1) and torch.equal(v2, v1)
    assert torch.equal(out2, out1)
    ref = oracle.paged_decode(case.q, k1.cpu(), v1.cpu(), case.block_table, case.seq_lens)
    assert_parity(out2, ref)


@pytest.mark.parametrize("b,hq,hkv,ctx,splits,dtype", [
    (1, 32, 8, 8192, 16, F16),    # 128 units of 16 tiles (the reference's workspace size)
    (2, 32, 8, 8192, 8, BF16),
    (8, 32, 8, 8192, 2, F16),
    (1, 16, 4, 20000, 32, BF16),  # partial last split
])
def test_split_with_the_reference_workspace(ext, gpu, b, hq, hkv, ctx, splits, dtype):
    case = make_case([ctx] * b, hq, hkv, 16, dtype, seed=ctx + splits)
    ws = torch.empty(b * hq * splits * 130, dtype=torch.float32, device=gpu)  # no sub-splits
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ext.paged_attention(case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu),
                        case.block_table.to(gpu), out, ws, ctx, 16, splits)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(out, ref)


def _draw(i):
    import random
    rng = random.Random(5000 + i)
    g = rng.choice([1, 2, 3, 4, 8, 16])
    hkv = rng.choice([1, 2, 4, 8])
    b = rng.randint(1, max(1, min(8, 128 // hkv)))  # at most 128 units
    op = ["paged", "masked", "indexed", "contiguous"][i % 4]
    ps = rng.choice([16, 32, 64])
    bucket = rng.randint(512, max(512, min(6000, 160000 // (b * hkv))))  # keeps the oracle fast
    lengths = [bucket] * b if op in ("paged", "contiguous") else \
        [bucket] + [rng.randint(0 if op != "paged" else 1, bucket) for _ in range(b - 1)]
    return op, g * hkv, hkv, ps, lengths, rng.choice([F16, BF16])


@pytest.mark.parametrize("i", range(48))
def test_random_few_unit_launches_without_workspace(ext, gpu, i):
    """Seeded draws of few-unit launches (at most 128 units of 16 or more tiles) with no
    workspace: every op, G up to 16, ragged and empty rows, pages 16-64, fp16 and bf16."""
    op, hq, hkv, ps, lengths, dtype = _draw(i)
    print(f"case {i}: {op} hq={hq} hkv={hkv} ps={ps} lengths={lengths} {dtype}", flush=True)
    b, bucket = len(lengths), max(lengths)
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    if op == "contiguous":
        gen = torch.Generator().manual_seed(i)
        q = torch.randn(b, hq, 128, generator=gen).to(dtype)
        k = torch.randn(b, hkv, bucket, 128, generator=gen).to(dtype)
        v = torch.randn(b, hkv, bucket, 128, generator=gen).to(dtype)
        ext.attention_contiguous(q.to(gpu), k.to(gpu), v.to(gpu), out, _empty(gpu), 1)
        torch.cuda.synchronize()
        assert_parity(out, torch.stack([oracle.sdpa_row(q[r], k[r], v[r]) for r in range(b)]))
        return
    case = make_case(lengths, hq, hkv, ps, dtype, seed=i, table_cols=-(-bucket // ps))
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    if op == "paged":
        ext.paged_attention(q, k, v, bt, out, _empty(gpu), bucket, ps, 1)
    elif op == "masked":
        ext.paged_attention_masked(q, k, v, bt, sl, out, _empty(gpu), bucket, ps, 1)
    else:
        idx = torch.arange(b, dtype=torch.int32, device=gpu).flip(0)
        ext.paged_attention_indexed(q, k, v, bt, sl, idx, idx, out, _empty(gpu), bucket, ps, 1)
        torch.cuda.synchronize()
        ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                                  case.seq_lens, idx.cpu(), idx.cpu(), b)
        assert_parity(out, ref)
        return
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(out, ref)
