"""Seeded random sweep at serving-like sizes, against the repack + fp32 SDPA oracle.

40 configurations with 20-256 rows whose lengths follow a heavy-tailed draw up to 20k
tokens (some 0), over the masked, indexed and work-queue ops (the work queue in both
schedules: beyond 64 rows the balanced kernels read the row lengths in 2-4 chunks of 64),
G in {1, 4, 8, 16, 32}, pages 16 and 32, fp16 and bf16, 1-20 splits.  Each case prints its
draw before it runs.
"""
import random

import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


def _draw(i):
    rng = random.Random(9000 + i)
    g = rng.choice([1, 4, 8, 16, 32])
    hkv = 1 if g == 32 else rng.choice([1, 2, 4, 8]) if g >= 8 else rng.choice([2, 4, 8])
    b = rng.choice([20, 48, 65, 100, 129, 200, 256])
    lengths = [0 if rng.random() < 0.03 else min(20000, int(rng.paretovariate(1.1) * 120))
               for _ in range(b)]
    if max(lengths) == 0:
        lengths[0] = 500
    return dict(op=["masked", "indexed", "workqueue", "workqueue"][i % 4], hq=g * hkv, hkv=hkv,
                ps=rng.choice([16, 32]), lengths=lengths, splits=rng.randint(1, 20),
                dtype=rng.choice([F16, BF16]), balanced=rng.random() < 0.7)


@pytest.mark.parametrize("i", range(40))
def test_random_large_configuration_matches_oracle(ext, gpu, i):
    c = _draw(i)
    op, hq, hkv, ps, lengths, dtype = (c[k] for k in ("op", "hq", "hkv", "ps", "lengths", "dtype"))
    b, bucket = len(lengths), max(lengths)
    print(f"case {i}: op {op} B {b} hq {hq} hkv {hkv} ps {ps} max len {bucket} "
          f"total {sum(lengths)} splits {c['splits']} {dtype} balanced {c['balanced']}", flush=True)
    splits = min(c["splits"], max(1, -(-bucket // 32)))
    case = make_case(lengths, hq, hkv, ps, dtype, seed=i, q_rows=b, table_cols=-(-bucket // ps))
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    if op in ("masked", "indexed"):
        floats = ext.split_workspace_floats(b, hq, hkv, bucket, splits) if splits > 1 else 0
        ws = torch.empty(max(floats, 1), dtype=torch.float32, device=gpu)
        if op == "masked":
            ext.paged_attention_masked(q, k, v, bt, sl, out, ws, bucket, ps, splits)
            ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                                      case.seq_lens)
        else:
            perm = torch.randperm(b, generator=torch.Generator().manual_seed(i)).to(torch.int32)
            ext.paged_attention_indexed(q, k, v, bt, sl, perm.to(gpu), perm.flip(0).contiguous().to(gpu),
                                        out, ws, bucket, ps, splits)
            ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                                      case.seq_lens, perm, perm.flip(0), b)
    else:
        meta = pkv_native.build_workqueue(lengths, list(range(b)), case.page_lists, ps, splits,
                                          False, hkv)
        t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
        floats = meta["total_partial_slots"] * hq * 130
        if c["balanced"]:
            floats = max(floats, pkv_native.workqueue_balanced_workspace_bytes(b, hq, hkv) // 4)
        ws = torch.empty(floats, dtype=torch.float32, device=gpu)
        counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
        ext.paged_attention_workqueue(q, k, v, t(meta["block_table"]), t(meta["seq_lens"]),
                                      t(meta["work_items"]), t(meta["split_offsets"]), counters,
                                      t(meta["q_indices"]), t(meta["out_indices"]), out, ws,
                                      meta["bucket_length"], ps, meta["total_partial_slots"], False)
        print("   schedule", ext.workqueue_schedule(b, hq, hkv, ps, floats, False), flush=True)
        ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                                  meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    torch.cuda.synchronize()
    assert_parity(out, ref)
