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


MAX_ABS = 2e-3   # north-star tolerance against the fp32 repack + SDPA oracle
MEAN_ABS = 3e-4  # the reference's mean gate (tests/smoke_test.cu:106)


def assert_parity(out, ref):
    """Gate of every parity test: max-abs 2e-3 and mean-abs 3e-4 against the fp32 oracle.

    bf16 outputs carry 8 significant bits, so a correctly rounded result can already sit
    half an output ulp from the fp32 value (3.9e-3 for |ref| in [1, 2)).  For bf16 the
    max-abs bound therefore adds half a bf16 ulp of |ref| (the kernel's own error stays
    within 2e-3) and the mean is taken against the oracle rounded to bf16.
    """
    got = out.float().cpu()
    mask = torch.isfinite(ref)
    assert torch.isfinite(got[mask]).all(), "non-finite output"
    diff = (got[mask] - ref[mask]).abs()
    if out.dtype == torch.bfloat16:
        mag = ref[mask].abs().clamp_min(2.0 ** -126)
        half_ulp = torch.exp2(torch.floor(torch.log2(mag)) - 8)
        excess = (diff - half_ulp).max().item()
        mean = (got[mask] - ref[mask].to(torch.bfloat16).float()).abs().mean().item()
        print(f"parity bf16: raw max-abs {diff.max().item():.3e}, max-abs beyond half an "
              f"output ulp {excess:.3e}, mean-abs vs bf16-rounded oracle {mean:.3e}, "
              f"raw mean-abs {diff.mean().item():.3e}")
        assert excess < MAX_ABS and mean < MEAN_ABS, (excess, mean, diff.max().item())
    else:
        mx, mean = diff.max().item(), diff.mean().item()
        print(f"parity {str(out.dtype).replace('torch.', '')}: max-abs {mx:.3e}, mean-abs {mean:.3e}")
        assert mx < MAX_ABS and mean < MEAN_ABS, (mx, mean)
