"""Seeded random sweep over the ops' argument space, against the repack + fp32 SDPA oracle.

The parametrised tests elsewhere pin chosen shapes; this sweep draws 512 configurations from
one seeded generator so that combinations no table lists are run too: every op (direct and
split paged_attention, masked, indexed with permuted and sparse output rows, the work queue
in both schedules and with the fused merge, contiguous K/V), G in {1, 2, 3, 4, 5, 8, 16,
24, 32}, page sizes 5-64, fp16 and bf16, 1-5 rows of 0-1500 tokens (0 only where a row may
be empty) and 1-8 splits.  Each case prints its draw before it runs, so a failure names it.
"""
import random

import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16
OPS = ["paged", "masked", "indexed", "workqueue", "contiguous"]
GROUPS = [1, 2, 3, 4, 5, 8, 16, 24, 32]


def _draw(i):
    rng = random.Random(1000 + i)
    op = OPS[i % len(OPS)]
    g = rng.choice(GROUPS)
    hkv = rng.choice([1, 2, 4]) if g >= 16 else rng.choice([1, 2, 4, 8])
    ps = rng.choice([16, 16, 32, 64, 8, 5])
    b = rng.randint(1, 5)
    empty_ok = op in ("masked", "indexed", "workqueue")
    lengths = [0 if empty_ok and rng.random() < 0.1 else rng.randint(1, 1500) for _ in range(b)]
    if max(lengths) == 0:
        lengths[0] = rng.randint(1, 1500)
    splits = rng.randint(1, 8)
    dtype = rng.choice([F16, BF16])
    return dict(op=op, hq=g * hkv, hkv=hkv, ps=ps, lengths=lengths, splits=splits, dtype=dtype,
                seed=i, balanced=rng.random() < 0.5, fused=rng.random() < 0.25)


def _ws(floats, gpu):
    return torch.empty(max(floats, 1), dtype=torch.float32, device=gpu)


@pytest.mark.parametrize("i", range(512))
def test_random_configuration_matches_oracle(ext, gpu, i):
    c = _draw(i)
    op, hq, hkv, ps, lengths, splits, dtype = (c[k] for k in ("op", "hq", "hkv", "ps", "lengths",
                                                               "splits", "dtype"))
    print(f"case {i}: {c}", flush=True)
    b = len(lengths)
    if op == "contiguous":
        n = max(lengths)
        splits = min(splits, max(1, -(-n // 32)))
        gen = torch.Generator().manual_seed(i)
        q = torch.randn(b, hq, 128, generator=gen).to(dtype)
        k = torch.randn(b, hkv, n, 128, generator=gen).to(dtype)
        v = torch.randn(b, hkv, n, 128, generator=gen).to(dtype)
        ref = torch.stack([oracle.sdpa_row(q[r], k[r], v[r]) for r in range(b)])
        out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
        floats = (ext.split_workspace_floats(b, hq, hkv, n, splits) if splits > 1
                  else ext.direct_workspace_floats(b, hq, hkv, n))
        ext.attention_contiguous(q.to(gpu), k.to(gpu), v.to(gpu), out, _ws(floats, gpu), splits)
        torch.cuda.synchronize()
        assert_parity(out, ref)
        return
    if op == "paged":
        lengths = [max(lengths)] * b  # the direct op reads `context` tokens of every row
    bucket = max(max(lengths), 1)
    splits = min(splits, max(1, -(-bucket // 32)))
    cols = -(-bucket // ps)
    case = make_case(lengths, hq, hkv, ps, dtype, seed=i, q_rows=b + 2, table_cols=cols)
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    if op == "paged":
        out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
        floats = (ext.split_workspace_floats(b, hq, hkv, bucket, splits) if splits > 1
                  else ext.direct_workspace_floats(b, hq, hkv, bucket))
        ext.paged_attention(q[:b].contiguous(), k, v, bt, out, _ws(floats, gpu), bucket, ps, splits)
        ref = oracle.paged_decode(case.q[:b], case.k_pages, case.v_pages, case.block_table,
                                  case.seq_lens)
    elif op == "masked":
        out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
        floats = ext.split_workspace_floats(b, hq, hkv, bucket, splits) if splits > 1 else 0
        ext.paged_attention_masked(q[:b].contiguous(), k, v, bt, sl, out, _ws(floats, gpu), bucket,
                                   ps, splits)
        ref = oracle.paged_decode(case.q[:b], case.k_pages, case.v_pages, case.block_table,
                                  case.seq_lens)
    elif op == "indexed":
        rng = random.Random(i)
        q_idx = torch.tensor(rng.sample(range(b + 2), b), dtype=torch.int32)
        o_idx = torch.tensor(rng.sample(range(b + 2), b), dtype=torch.int32)
        out = torch.full((b + 2, hq, 128), 7.0, dtype=dtype, device=gpu)
        floats = ext.split_workspace_floats(b, hq, hkv, bucket, splits) if splits > 1 else 0
        ext.paged_attention_indexed(q, k, v, bt, sl, q_idx.to(gpu), o_idx.to(gpu), out,
                                    _ws(floats, gpu), bucket, ps, splits)
        ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                                  case.seq_lens, q_idx, o_idx, b + 2)
        untouched = [r for r in range(b + 2) if r not in o_idx.tolist()]
        torch.cuda.synchronize()
        assert torch.all(out[untouched].float().cpu() == 7.0)
    else:
        ids = list(range(b))
        meta = pkv_native.build_workqueue(lengths, ids, case.page_lists, ps, splits, False, hkv)
        t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
        floats = meta["total_partial_slots"] * hq * 130
        if c["balanced"]:
            floats = max(floats, pkv_native.workqueue_balanced_workspace_bytes(b, hq, hkv) // 4)
        out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
        counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
        ext.paged_attention_workqueue(q, k, v, t(meta["block_table"]), t(meta["seq_lens"]),
                                      t(meta["work_items"]), t(meta["split_offsets"]), counters,
                                      t(meta["q_indices"]), t(meta["out_indices"]), out,
                                      _ws(floats, gpu), meta["bucket_length"], ps,
                                      meta["total_partial_slots"], c["fused"])
        ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                                  meta["seq_lens"], meta["q_indices"], meta["out_indices"])
        torch.cuda.synchronize()
        assert int(counters.abs().sum()) == 0
    torch.cuda.synchronize()
    assert_parity(out, ref)
