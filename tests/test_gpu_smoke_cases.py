"""The reference's own correctness cases (tests/smoke_test.cu:486-493) on the HIP engine.

Inputs are regenerated exactly (glibc srand(42)/rand(), quantised to fp16) and checked
against the CRC in tests/golden/smoke_expected.npz; the expected outputs there are the
reference's fp32 CPU attention (smoke_test.cu:35-74).  The reference's contiguous cases
(0-5) run through the contiguous-layout op, as they do in the reference
(persistentkv_dispatch / persistentkv_split_dispatch, smoke_test.cu:155-163), through the
query-head baseline (smoke_test.cu:176-192 checks it on case 0) and through the paged op
with an identity table of 16-token pages; the paged cases use the reference's reversed
physical page order (smoke_test.cu:239-258).  Gate: max-abs < 2e-3 and mean-abs < 3e-4
(smoke_test.cu:106, :205).
"""
import os
import zlib

import numpy as np
import pytest
import torch

from conftest import MAX_ABS, MEAN_ABS
from oracle import native

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "smoke_expected.npz")


def to_pages(k, page_size, reverse):
    """[B, Hkv, N, d] -> pool [B*ppb, Hkv, ps, d] and table [B, ppb]."""
    b, hkv, n, d = k.shape
    ppb = -(-n // page_size)
    pool = np.zeros((b * ppb, hkv, page_size, d), dtype=k.dtype)
    table = np.zeros((b, ppb), dtype=np.int32)
    for row in range(b):
        for logical in range(ppb):
            physical = row * ppb + (ppb - 1 - logical if reverse else logical)
            table[row, logical] = physical
            lo, hi = logical * page_size, min(n, (logical + 1) * page_size)
            pool[physical, :, : hi - lo] = k[row, :, lo:hi]
    return pool, table


@pytest.mark.parametrize("index", range(8))
def test_reference_smoke_case(ext, gpu, index):
    golden = np.load(GOLDEN)
    b, hq, hkv, n, splits, page_size = (int(x) for x in golden[f"shape_{index}"])
    q, k, v = native.smoke_inputs(index)
    q16, k16, v16 = q.astype(np.float16), k.astype(np.float16), v.astype(np.float16)
    assert zlib.crc32(q16.tobytes() + k16.tobytes() + v16.tobytes()) == int(golden[f"crc_{index}"][0])
    reverse = page_size != 0
    ps = page_size or 16
    kp, table = to_pages(k16, ps, reverse)
    vp, _ = to_pages(v16, ps, reverse)
    dev = gpu
    out = torch.full((b, hq, 128), float("nan"), dtype=torch.float16, device=dev)
    ws = torch.empty(b * hq * splits * 130 if splits > 1 else 0, dtype=torch.float32, device=dev)
    ext.paged_attention(torch.from_numpy(q16).to(dev), torch.from_numpy(kp).to(dev),
                        torch.from_numpy(vp).to(dev), torch.from_numpy(table).to(dev), out, ws, n,
                        ps, splits)
    torch.cuda.synchronize()
    diff = np.abs(out.float().cpu().numpy() - golden[f"expected_{index}"])
    print(f"smoke case {index} B={b} Hq={hq} Hkv={hkv} N={n} splits={splits} page={ps} "
          f"max_err={diff.max():.2e} mean_err={diff.mean():.2e}")
    assert diff.max() < MAX_ABS and diff.mean() < MEAN_ABS


def _check(out, golden, index, label):
    diff = np.abs(out.float().cpu().numpy() - golden[f"expected_{index}"])
    print(f"smoke case {index} {label} max_err={diff.max():.2e} mean_err={diff.mean():.2e}")
    assert diff.max() < MAX_ABS and diff.mean() < MEAN_ABS


@pytest.mark.parametrize("index", range(6))
def test_reference_smoke_case_contiguous_layout(ext, gpu, index):
    golden = np.load(GOLDEN)
    b, hq, hkv, n, splits, page_size = (int(x) for x in golden[f"shape_{index}"])
    assert page_size == 0  # cases 0-5 are contiguous in the reference
    q, k, v = (torch.from_numpy(x.astype(np.float16)).to(gpu) for x in native.smoke_inputs(index))
    out = torch.full((b, hq, 128), float("nan"), dtype=torch.float16, device=gpu)
    ws = torch.empty(b * hq * splits * 130 if splits > 1 else 0, dtype=torch.float32, device=gpu)
    ext.attention_contiguous(q, k, v, out, ws, splits)
    base = torch.full_like(out, float("nan"))
    ext.attention_query_head_baseline(q, k, v, base)
    torch.cuda.synchronize()
    _check(out, golden, index, f"contiguous splits={splits}")
    _check(base, golden, index, "query-head baseline")
