"""Seeded paged-KV inputs shared by the GPU parity tests (CPU tensors)."""
from __future__ import annotations

from dataclasses import dataclass

import torch

from oracle import attention as oracle


@dataclass
class PagedCase:
    q: torch.Tensor            # [q_rows, Hq, 128]
    k_pages: torch.Tensor      # [pages, Hkv, ps, 128]
    v_pages: torch.Tensor
    block_table: torch.Tensor  # [B, max_pages] int32
    seq_lens: torch.Tensor     # [B] int32
    page_lists: list
    page_size: int


def make_case(lengths, hq, hkv, page_size, dtype=torch.float16, seed=0, table="random",
              extra_pages=3, q_rows=None, table_cols=None):
    """Pages for each row are drawn from one pool; ``table`` picks how: "random"
    (a seeded permutation), "reversed" (each row's pages in reverse physical order, as in
    tests/smoke_test.cu:239-258), "contiguous" (identity) or "canonical"
    ((405p + 17) mod 2L, benchmark_native_paged_baselines.py:38-42; one row)."""
    gen = torch.Generator().manual_seed(seed)
    pages = [max(1, -(-n // page_size)) for n in lengths]
    if table == "canonical":
        assert len(lengths) == 1
        rows = [oracle.canonical_block_table(pages[0] * page_size, page_size)]
        pool = 2 * pages[0]
    else:
        pool = sum(pages) + extra_pages
        order = (torch.randperm(pool, generator=gen).tolist() if table == "random"
                 else list(range(pool)))
        rows, cur = [], 0
        for p in pages:
            row = order[cur:cur + p]
            rows.append(row[::-1] if table == "reversed" else row)
            cur += p
    cols = table_cols or max(pages)
    bt = torch.tensor([r + [r[-1]] * (cols - len(r)) for r in rows], dtype=torch.int32)
    k = torch.randn(pool, hkv, page_size, 128, generator=gen).to(dtype)
    v = torch.randn(pool, hkv, page_size, 128, generator=gen).to(dtype)
    q = torch.randn(q_rows or len(lengths), hq, 128, generator=gen).to(dtype)
    return PagedCase(q, k, v, bt, torch.tensor(lengths, dtype=torch.int32), rows, page_size)


def errors(out, ref):
    """(max-abs, mean-abs) over the finite reference entries."""
    out = out.float().cpu()
    mask = torch.isfinite(ref)
    diff = (out[mask] - ref[mask]).abs()
    return diff.max().item(), diff.mean().item()
