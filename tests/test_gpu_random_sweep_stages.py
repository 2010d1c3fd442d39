"""Seeded random sweep over the work-queue op's stage entry points.

128 configurations (G 1-32, pages 5-64, fp16 and bf16, fp8 K/V on a third of the draws
with pages of a multiple of 16, 1-6 rows of 0-3000 tokens, 1-12 splits, both schedules):
- paged_attention_workqueue_stage(1) then (2) on one workspace equals the combined op
  (the same schedule, chosen by the workspace size) bit for bit;
- the reference's two stages, workqueue_decode then workqueue_merge (one workgroup per
  item, the reference's partial-state layout), equal the combined op with the fused
  merge (the same schedule and partial states) bit for bit;
- the combined op matches the repack + fp32 SDPA oracle.
Each case prints its draw before it runs.
"""
import random

import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16, BF16, F8 = torch.float16, torch.bfloat16, torch.float8_e4m3fn


def _draw(i):
    rng = random.Random(7000 + i)
    g = rng.choice([1, 2, 3, 4, 8, 16, 24, 32])
    hkv = rng.choice([1, 2, 4]) if g >= 16 else rng.choice([1, 2, 4, 8])
    fp8 = i % 3 == 0
    b = rng.randint(1, 6)
    lengths = [0 if rng.random() < 0.08 else rng.randint(1, 3000) for _ in range(b)]
    if max(lengths) == 0:
        lengths[0] = rng.randint(1, 3000)
    return dict(hq=g * hkv, hkv=hkv, ps=rng.choice([16, 32, 64] if fp8 else [16, 32, 64, 8, 5]),
                lengths=lengths, splits=rng.randint(1, 12), dtype=rng.choice([F16, BF16]),
                fp8=fp8, scale=rng.choice([0.03, 0.06]), balanced=rng.random() < 0.6)


@pytest.mark.parametrize("i", range(128))
def test_random_stages_equal_combined(ext, gpu, i):
    c = _draw(i)
    print(f"case {i}: {c}", flush=True)
    hq, hkv, ps, lengths, dtype, fp8, sc = (c[k] for k in ("hq", "hkv", "ps", "lengths", "dtype",
                                                          "fp8", "scale"))
    b = len(lengths)
    case = make_case(lengths, hq, hkv, ps, dtype, seed=i)
    meta = pkv_native.build_workqueue(lengths, list(range(b)), case.page_lists, ps, c["splits"],
                                      False, hkv)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    bt, sl, wi, so, qi, oi = (t(meta[k]) for k in ("block_table", "seq_lens", "work_items",
                                                   "split_offsets", "q_indices", "out_indices"))
    slots, bucket = meta["total_partial_slots"], meta["bucket_length"]
    floats = slots * hq * 130
    if c["balanced"]:
        floats = max(floats, pkv_native.workqueue_balanced_workspace_bytes(b, hq, hkv) // 4)
    q = case.q.to(gpu)
    if fp8:
        k = (case.k_pages.float() / sc).clamp(-448, 448).to(F8).to(gpu)
        v = (case.v_pages.float() / sc).clamp(-448, 448).to(F8).to(gpu)
    else:
        k, v = case.k_pages.to(gpu), case.v_pages.to(gpu)
    quant = (sc, sc) if fp8 else ()

    def fresh():
        return (torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu),
                torch.empty(floats, dtype=torch.float32, device=gpu))

    def combined(fused):
        out, ws = fresh()
        counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
        op = ext.paged_attention_workqueue_fp8 if fp8 else ext.paged_attention_workqueue
        op(q, k, v, bt, sl, wi, so, counters, qi, oi, out, ws, bucket, ps, slots, fused, *quant)
        torch.cuda.synchronize()
        assert int(counters.abs().sum()) == 0
        return out

    one = combined(False)
    out, ws = fresh()
    for stage in (1, 2):
        ext.paged_attention_workqueue_stage(stage, q, k, v, bt, sl, wi, so, qi, oi, out, ws, bucket,
                                            ps, slots, fp8, sc, sc)
    torch.cuda.synchronize()
    assert torch.equal(out, one)
    ref_out, ref_ws = fresh()
    if fp8:
        ext.workqueue_decode_fp8(q, k, v, bt, sl, wi, so, qi, ref_ws, bucket, ps, slots, sc, sc)
    else:
        ext.workqueue_decode(q, k, v, bt, sl, wi, so, qi, ref_ws, bucket, ps, slots)
    ext.workqueue_merge(sl, so, oi, ref_out, ref_ws, slots)
    torch.cuda.synchronize()
    assert torch.equal(ref_out, combined(True))
    kd = oracle.dequantize_e4m3(k.cpu(), sc) if fp8 else case.k_pages
    vd = oracle.dequantize_e4m3(v.cpu(), sc) if fp8 else case.v_pages
    ref = oracle.paged_decode(case.q, kd, vd, meta["block_table"], meta["seq_lens"],
                              meta["q_indices"], meta["out_indices"])
    assert_parity(one, ref)
