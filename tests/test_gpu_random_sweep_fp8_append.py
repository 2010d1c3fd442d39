"""Seeded random sweep over the fp8 and fused-append entry points.

256 configurations from one seeded generator over paged_attention_indexed_fp8,
paged_attention_workqueue_fp8 and the five ops with the KV-cache append fused in (masked,
indexed and work queue on 2-byte pools, indexed and work queue on fp8 pools): G 1-32,
page sizes 5-64 (fp8 pools: 16, 32, 64, as the fp8 ops require), fp16 and bf16
activations, 1-5 rows of 0-1500 tokens, 1-8 splits, both work-queue schedules and the
fused merge.  Each case checks
- the fused op against append_kv (append_kv_fp8) followed by the plain op: pools and
  output bit for bit;
- the pools against the oracle's append (fp8 pools: the new token's bytes are
  quantize_e4m3 of it);
- the output against the repack + fp32 SDPA oracle on the resulting pools (dequantised
  for fp8).
Each case prints its draw before it runs, so a failure names it.
"""
import random

import numpy as np
import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16, BF16, F8 = torch.float16, torch.bfloat16, torch.float8_e4m3fn
OPS = ["indexed_fp8", "workqueue_fp8", "masked_append", "indexed_append", "workqueue_append",
       "indexed_fp8_append", "workqueue_fp8_append"]
GROUPS = [1, 2, 3, 4, 5, 8, 16, 24, 32]


def _draw(i):
    rng = random.Random(5000 + i)
    g = rng.choice(GROUPS)
    hkv = rng.choice([1, 2, 4]) if g >= 16 else rng.choice([1, 2, 4, 8])
    b = rng.randint(1, 5)
    lengths = [0 if rng.random() < 0.08 else rng.randint(1, 1500) for _ in range(b)]
    if max(lengths) == 0:
        lengths[0] = rng.randint(1, 1500)
    op = OPS[i % len(OPS)]
    sizes = [16, 32, 64] if "fp8" in op else [16, 16, 32, 64, 8, 5]  # fp8 pools: multiples of 16
    return dict(op=op, hq=g * hkv, hkv=hkv, ps=rng.choice(sizes),
                lengths=lengths, splits=rng.randint(1, 8), dtype=rng.choice([F16, BF16]),
                scale=rng.choice([0.02, 0.05, 0.1]), balanced=rng.random() < 0.5,
                fused=rng.random() < 0.25)


def _quantise(x, scale):
    return (x.float() / scale).clamp(-448.0, 448.0).to(F8)


@pytest.mark.parametrize("i", range(256))
def test_random_fp8_and_append_configuration(ext, gpu, i):
    c = _draw(i)
    print(f"case {i}: {c}", flush=True)
    op, hq, hkv, ps, lengths, dtype, sc = (c[k] for k in ("op", "hq", "hkv", "ps", "lengths",
                                                          "dtype", "scale"))
    fp8, append, queue = "fp8" in op, op.endswith("_append"), op.startswith("workqueue")
    b, bucket = len(lengths), max(lengths)
    splits = min(c["splits"], max(1, -(-bucket // 32)))
    case = make_case(lengths, hq, hkv, ps, dtype, seed=i, q_rows=b + 2, table_cols=-(-bucket // ps))
    gen = torch.Generator().manual_seed(100 + i)
    kn = torch.randn(b, hkv, 128, generator=gen).to(dtype)
    vn = torch.randn(b, hkv, 128, generator=gen).to(dtype)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    q = case.q.to(gpu)
    if queue:
        meta = pkv_native.build_workqueue(lengths, list(range(b)), case.page_lists, ps, splits, False,
                                          hkv)
        bt, sl = t(meta["block_table"]), t(meta["seq_lens"])
        floats = meta["total_partial_slots"] * hq * 130
        if c["balanced"]:
            floats = max(floats, pkv_native.workqueue_balanced_workspace_bytes(b, hq, hkv) // 4)
        q_idx, o_idx, out_rows = meta["q_indices"], meta["out_indices"], b
    else:
        bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
        floats = ext.split_workspace_floats(b, hq, hkv, bucket, splits) if splits > 1 else 0
        rng = random.Random(i)
        q_idx = torch.tensor(rng.sample(range(b + 2), b), dtype=torch.int32)
        o_idx = torch.tensor(rng.sample(range(b + 2), b), dtype=torch.int32)
        out_rows = b + 2
        if op == "masked_append":
            q_idx, o_idx, out_rows = torch.arange(b, dtype=torch.int32), torch.arange(b, dtype=torch.int32), b

    def run(fused_append):
        if fp8:
            k, v = _quantise(case.k_pages, sc).to(gpu), _quantise(case.v_pages, sc).to(gpu)
        else:
            k, v = case.k_pages.to(gpu), case.v_pages.to(gpu)
        out = torch.full((out_rows, hq, 128), 7.0, dtype=dtype, device=gpu)
        ws = torch.empty(max(floats, 1), dtype=torch.float32, device=gpu)
        counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
        new = (kn.to(gpu), vn.to(gpu))
        if append and not fused_append:
            if fp8:
                ext.append_kv_fp8(*new, k, v, bt, sl, sc, sc)
            else:
                ext.append_kv(*new, k, v, bt, sl)
        if queue:
            args = (q, k, v, bt, sl, t(meta["work_items"]), t(meta["split_offsets"]), counters,
                    t(q_idx), t(o_idx), out, ws, meta["bucket_length"], ps,
                    meta["total_partial_slots"], c["fused"])
        elif op == "masked_append":
            args = (q[:b].contiguous(), k, v, bt, sl, out, ws, bucket, ps, splits)
        else:
            args = (q, k, v, bt, sl, t(q_idx), t(o_idx), out, ws, bucket, ps, splits)
        if fp8:
            args = args + (sc, sc)
        name = {"indexed": "paged_attention_indexed", "workqueue": "paged_attention_workqueue",
                "masked": "paged_attention_masked"}[op.split("_")[0]] + ("_fp8" if fp8 else "")
        if append and fused_append:
            getattr(ext, name + "_append")(*args, *new)
        else:
            getattr(ext, name)(*args)
        torch.cuda.synchronize()
        assert int(counters.abs().sum()) == 0
        return out.cpu(), k.cpu(), v.cpu()

    out, k, v = run(append)
    if append:
        out0, k0, v0 = run(False)
        bits = (lambda x: x.view(torch.uint8)) if fp8 else (lambda x: x)
        assert torch.equal(bits(k), bits(k0)) and torch.equal(bits(v), bits(v0))
        assert torch.equal(out, out0)
        table = bt.cpu()
        for r, n in enumerate(lengths):  # the appended slots, against the oracle's append
            if n <= 0:
                continue
            page, slot = int(table[r, (n - 1) // ps]), (n - 1) % ps
            if fp8:
                for x, new in ((k, kn), (v, vn)):
                    got = x.view(torch.uint8)[page, :, slot].numpy()
                    assert np.array_equal(got, oracle.quantize_e4m3(new[r].float().numpy(), sc))
        if not fp8:
            k_ref, v_ref = oracle.append_kv(case.k_pages, case.v_pages, table, sl.cpu(), kn, vn)
            assert torch.equal(k, k_ref) and torch.equal(v, v_ref)
    if fp8:
        k, v = oracle.dequantize_e4m3(k, sc), oracle.dequantize_e4m3(v, sc)
    ref = oracle.paged_decode(case.q if out_rows > b or queue else case.q[:b], k, v, bt.cpu(),
                              sl.cpu(), q_idx if op != "masked_append" else None,
                              o_idx if op != "masked_append" else None,
                              out_rows if op != "masked_append" else None)
    assert_parity(out, ref)
    if not queue and op != "masked_append":
        untouched = [r for r in range(out_rows) if r not in o_idx.tolist()]
        assert torch.all(out[untouched].float() == 7.0)
