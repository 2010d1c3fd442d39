"""Scores that keep rising, falling or spiking along a row: the decode's running-max rescale.

The decode raises a head's running max only when a tile's scores pass it by more than 8
(log2 units) and then rescales the accumulated output, sum and partial max by
2^(old - new).  With N(0, 1) inputs that almost never happens after the first tile, so
here each KV head's keys are a ramp along the row in the direction of one of its query
heads: that head's scores rise by ~10 log2 units per 32-token tile, so every tile
rescales; the group's other heads see rising, falling or flat scores depending on their
angle to it; "spikes" plants a few tokens whose scores jump by ~40-80 log2 units above
the rest.  Every schedule is run (direct, the whole-line direct launch, split, masked,
indexed, the work queue per item, balanced and fused) for G = 4, 8 and 32, fp16 and bf16,
against the repack + fp32 SDPA oracle at the parity bar.
"""
import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16, BF16 = torch.float16, torch.bfloat16


def _plant(case, pattern, seed):
    """Rewrites the keys of every row in place (pages are not shared between rows)."""
    gen = torch.Generator().manual_seed(seed)
    hq, hkv, ps = case.q.shape[1], case.k_pages.shape[1], case.page_size
    g = hq // hkv
    k = case.k_pages.float()
    for r, n in enumerate(case.seq_lens.tolist()):
        for kvh in range(hkv):
            u = case.q[r, kvh * g].float()
            u = u / u.norm() * 128 ** 0.5  # |u| = sqrt(128): u.k ~ scale * 128
            t = torch.arange(n, dtype=torch.float32)
            if pattern == "rising":
                scale = 0.02 * t
            elif pattern == "falling":
                scale = 0.02 * (n - 1 - t)
            else:  # spikes on a flat row
                scale = torch.zeros(n)
                for p in torch.randint(0, n, (max(1, n // 300),), generator=gen).tolist():
                    scale[p] = 3.0 + 3.0 * torch.rand(1, generator=gen).item()
            rows = scale[:, None] * u[None, :] + 0.3 * torch.randn(n, 128, generator=gen)
            for tok in range(n):
                page = int(case.block_table[r, tok // ps])
                k[page, kvh, tok % ps] = rows[tok]
    case.k_pages = k.to(case.k_pages.dtype)


def _ws(floats, gpu):
    return torch.empty(max(floats, 0), dtype=torch.float32, device=gpu)


CASES = [  # (op, lengths, hq, hkv, page_size, splits, dtype)
    ("paged", [2048], 32, 8, 16, 1, F16),           # no workspace: the whole-line direct launch
    ("paged", [1500, 1500], 32, 8, 16, 1, BF16),    # direct, split inside
    ("paged", [1000], 32, 1, 32, 4, BF16),          # G = 32, split
    ("masked", [40, 1200, 700], 32, 4, 16, 3, F16),  # G = 8
    ("indexed", [900, 33, 1400], 32, 8, 16, 1, BF16),
    ("queue", [300, 1500, 64, 900], 32, 8, 16, 6, F16),
    ("queue", [300, 1500, 64, 900], 32, 1, 32, 6, BF16),  # G = 32: per item
    ("balanced", [300, 1500, 64, 900], 32, 8, 16, 6, BF16),
    ("fused", [1200, 500], 32, 4, 16, 5, F16),
]


@pytest.mark.parametrize("pattern", ["rising", "falling", "spikes"])
@pytest.mark.parametrize("op,lengths,hq,hkv,ps,splits,dtype", CASES)
def test_running_max_rescale(ext, gpu, pattern, op, lengths, hq, hkv, ps, splits, dtype):
    print(f"{op} {pattern} lengths={lengths} G={hq // hkv} {dtype}", flush=True)
    case = make_case(lengths, hq, hkv, ps, dtype, seed=sum(lengths) + splits)
    _plant(case, pattern, seed=len(lengths))
    b, bucket = len(lengths), max(lengths)
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    bt, sl = case.block_table.to(gpu), case.seq_lens.to(gpu)
    out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    if op == "paged":
        floats = ext.split_workspace_floats(b, hq, hkv, bucket, splits) if splits > 1 else (
            0 if b == 1 else ext.direct_workspace_floats(b, hq, hkv, bucket))
        ext.paged_attention(q, k, v, bt, out, _ws(floats, gpu), bucket, ps, splits)
    elif op == "masked":
        ext.paged_attention_masked(q, k, v, bt, sl, out, _ws(b * hq * splits * 130, gpu), bucket,
                                   ps, splits)
    elif op == "indexed":
        idx = torch.arange(b, dtype=torch.int32, device=gpu)
        ext.paged_attention_indexed(q, k, v, bt, sl, idx, idx, out, _ws(0, gpu), bucket, ps, splits)
    else:
        meta = pkv_native.build_workqueue(lengths, list(range(b)), case.page_lists, ps, splits,
                                          False, hkv)
        t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
        floats = meta["total_partial_slots"] * hq * 130
        if op == "balanced":
            floats = max(floats, pkv_native.workqueue_balanced_workspace_bytes(b, hq, hkv) // 4)
            assert pkv_native.workqueue_schedule(b, hq, hkv, ps, floats * 4) == 1
        counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
        ext.paged_attention_workqueue(q, k, v, t(meta["block_table"]), t(meta["seq_lens"]),
                                      t(meta["work_items"]), t(meta["split_offsets"]), counters,
                                      t(meta["q_indices"]), t(meta["out_indices"]), out,
                                      _ws(floats, gpu), meta["bucket_length"], ps,
                                      meta["total_partial_slots"], op == "fused")
    torch.cuda.synchronize()
    assert_parity(out, ref)
