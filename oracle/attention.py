"""Reference outputs for paged decode attention (CPU; test infrastructure only).

The reference defines correctness as "gather the row's pages, repack them to contiguous
K/V, run fp32 scaled-dot-product attention with GQA" (tests/benchmark_torch_paged_sdpa.py
:90-103 for the HND page layout, tests/benchmark_native_paged_baselines.py:83-94 and
:268-287 for the SDPA call).  This module restates that, plus an fp64 brute force and
the split-K partial states / log-sum-exp merge of kernels/persistentkv_attention.cuh.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

HEAD_DIM = 128
TILE = 32                       # kernels/persistentkv_attention.cuh:28
SCALE = 1.0 / math.sqrt(HEAD_DIM)  # cuh:944
NEG_FLT_MAX = -np.finfo(np.float32).max


def _cpu(t):
    return t.detach().cpu() if isinstance(t, torch.Tensor) else torch.as_tensor(t)


def gather_row(k_pages, v_pages, table_row, length):
    """Contiguous ``[Hkv, length, 128]`` K and V of one row.

    Follows benchmark_torch_paged_sdpa.py:90-103: ``index_select`` over the page axis of
    the ``[pages, Hkv, page_size, 128]`` pool, permute to ``[Hkv, pages, page_size, 128]``,
    flatten the tokens and trim to the row length.
    """
    k_pages, v_pages = _cpu(k_pages), _cpu(v_pages)
    hkv, ps = k_pages.shape[1], k_pages.shape[2]
    n_pages = -(-int(length) // ps)
    idx = _cpu(table_row)[:n_pages].long()
    k = k_pages.index_select(0, idx).permute(1, 0, 2, 3).reshape(hkv, n_pages * ps, HEAD_DIM)
    v = v_pages.index_select(0, idx).permute(1, 0, 2, 3).reshape(hkv, n_pages * ps, HEAD_DIM)
    return k[:, :length], v[:, :length]


def sdpa_row(q_row, k, v):
    """fp32 SDPA with ``enable_gqa`` for one query row: q ``[Hq,128]``, k/v ``[Hkv,L,128]``.

    benchmark_native_paged_baselines.py:83-94 (query head h reads KV head h // G).
    """
    qf = _cpu(q_row).float().unsqueeze(0).unsqueeze(2)
    kf = _cpu(k).float().unsqueeze(0)
    vf = _cpu(v).float().unsqueeze(0)
    out = F.scaled_dot_product_attention(qf, kf, vf, is_causal=False, enable_gqa=True)
    return out.squeeze(0).squeeze(1)


def paged_decode(q, k_pages, v_pages, block_table, seq_lens, q_indices=None,
                 out_indices=None, out_rows=None):
    """Reference result of the four ops as float32 ``[out_rows, Hq, 128]``.

    Row ``b`` reads query row ``q_indices[b]`` (default ``b``), attends to its first
    ``seq_lens[b]`` tokens and writes output row ``out_indices[b]`` (default ``b``).
    Rows that no ``b`` writes stay NaN; zero-length rows are 0 (the merge's L == 0 rule,
    cuh:749-750).
    """
    q = _cpu(q)
    block_table = _cpu(block_table)
    seq_lens = [int(x) for x in _cpu(seq_lens).tolist()]
    batch = len(seq_lens)
    q_idx = list(range(batch)) if q_indices is None else [int(x) for x in _cpu(q_indices).tolist()]
    o_idx = list(range(batch)) if out_indices is None else [int(x) for x in _cpu(out_indices).tolist()]
    rows = batch if out_rows is None else out_rows
    hq = q.shape[1]
    out = torch.full((rows, hq, HEAD_DIM), float("nan"), dtype=torch.float32)
    for b in range(batch):
        if seq_lens[b] <= 0:
            out[o_idx[b]] = 0.0
            continue
        k, v = gather_row(k_pages, v_pages, block_table[b], seq_lens[b])
        out[o_idx[b]] = sdpa_row(q[q_idx[b]], k, v)
    return out


def attention_fp64(q_row, k, v):
    """Textbook softmax attention in float64: q ``[Hq,128]``, k/v ``[Hkv,L,128]``."""
    q = np.asarray(_cpu(q_row).double().numpy())
    k = np.asarray(_cpu(k).double().numpy())
    v = np.asarray(_cpu(v).double().numpy())
    hq, hkv = q.shape[0], k.shape[0]
    g = hq // hkv
    out = np.zeros((hq, HEAD_DIM))
    for h in range(hq):
        s = k[h // g] @ q[h] * SCALE
        s = s - s.max()
        p = np.exp(s)
        out[h] = (p @ v[h // g]) / p.sum()
    return out


def split_bounds(total_tiles, num_splits):
    """Row-local split ranges in 32-token tiles, cuh:330-337."""
    return [((total_tiles * s) // num_splits, (total_tiles * (s + 1)) // num_splits)
            for s in range(num_splits)]


def split_partials(q_row, k, v, ranges):
    """Partial states ``(m, l, acc)`` of each tile range, float64.

    ``m`` is the max of ``score * scale`` over the range (natural-log units), ``l`` is
    ``sum exp(s - m)`` and ``acc`` is ``sum exp(s - m) v``; an empty range gives the
    neutral state ``(-FLT_MAX, 0, 0)`` (cuh:340-363, :615-632).  Shapes ``[Hq, S]``,
    ``[Hq, S]``, ``[Hq, S, 128]``.
    """
    q = np.asarray(_cpu(q_row).double().numpy())
    k = np.asarray(_cpu(k).double().numpy())
    v = np.asarray(_cpu(v).double().numpy())
    hq, hkv, length = q.shape[0], k.shape[0], k.shape[1]
    g = hq // hkv
    n = len(ranges)
    m = np.full((hq, n), float(NEG_FLT_MAX))
    l = np.zeros((hq, n))
    acc = np.zeros((hq, n, HEAD_DIM))
    for h in range(hq):
        s_all = k[h // g] @ q[h] * SCALE
        for i, (tb, te) in enumerate(ranges):
            lo, hi = tb * TILE, min(te * TILE, length)
            if hi <= lo:
                continue
            s = s_all[lo:hi]
            m[h, i] = s.max()
            p = np.exp(s - m[h, i])
            l[h, i] = p.sum()
            acc[h, i] = p @ v[h // g, lo:hi]
    return m, l, acc


def lse_merge(m, l, acc):
    """Log-sum-exp merge over the last split axis (cuh:719-751); 0 where L == 0."""
    big_m = m.max(axis=-1, keepdims=True)
    w = np.exp(m - big_m)
    big_l = (w * l).sum(axis=-1)
    a = (w[..., None] * acc).sum(axis=-2)
    with np.errstate(invalid="ignore", divide="ignore"):
        out = np.where(big_l[..., None] > 0, a / big_l[..., None], 0.0)
    return out


def canonical_block_table(context, page_size=16):
    """``(405 * p + 17) mod (2 * pages)`` (benchmark_native_paged_baselines.py:38-42)."""
    logical = context // page_size
    physical = logical * 2
    return [(405 * p + 17) % physical for p in range(logical)]


def e4m3_value(code):
    """OCP FP8 E4M3 (the `float8_e4m3fn` format) decoded from the format's definition
    (OCP 8-bit Floating Point Specification v1.0): sign bit, 4 exponent bits with bias 7,
    3 mantissa bits; exponent 0 is subnormal (2^-6 * m/8); no infinities; only
    S.1111.111 is NaN, so the largest finite value is 1.75 * 2^8 = 448.  The reference has
    no fp8 path; this pins the dequantisation the fp8 K/V ops are checked against."""
    sign = -1.0 if code & 0x80 else 1.0
    exponent, mantissa = (code >> 3) & 0xF, code & 0x7
    if exponent == 0xF and mantissa == 0x7:
        return float("nan")
    if exponent == 0:
        return sign * 2.0 ** -6 * (mantissa / 8.0)
    return sign * 2.0 ** (exponent - 7) * (1.0 + mantissa / 8.0)


E4M3_TABLE = np.array([e4m3_value(c) for c in range(256)], dtype=np.float32)


def dequantize_e4m3(pages, scale):
    """fp32 ``scale * e4m3(pages)`` for a tensor of e4m3 bytes (``float8_e4m3fn`` or
    ``uint8``)."""
    codes = _cpu(pages).contiguous().view(torch.uint8).numpy()
    return torch.from_numpy(E4M3_TABLE[codes] * np.float32(scale))


# Positive finite e4m3 codes 0x00..0x7e in increasing value (the format is monotone over
# them), for the nearest-value search below.
_E4M3_POS_CODES = np.arange(0x7F, dtype=np.int64)
_E4M3_POS_VALUES = E4M3_TABLE[:0x7F].astype(np.float64)


def quantize_e4m3(x, scale):
    """e4m3 bytes (uint8 numpy array) of ``clamp(x / scale, -448, 448)`` rounded to the
    nearest representable value, ties to the even code: the conversion the fp8 K/V
    producers use (torch's ``float8_e4m3fn`` cast after the clamp).  The quotient is taken
    in fp32.  NaN keeps its sign (0x7f, 0xff).  The reference has no fp8 path.

    Found by searching the decoded value table rather than by bit manipulation, so the
    check of a bit-level encoder against it is independent."""
    with np.errstate(over="ignore", invalid="ignore"):
        y = np.asarray(x, dtype=np.float32) / np.float32(scale)
    sign = np.signbit(y).astype(np.uint8) << 7
    a = np.minimum(np.abs(y).astype(np.float64), 448.0)
    hi = np.clip(np.searchsorted(_E4M3_POS_VALUES, a, side="left"), 0, 0x7E)
    lo = np.clip(hi - 1, 0, 0x7E)
    d_lo, d_hi = a - _E4M3_POS_VALUES[lo], _E4M3_POS_VALUES[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (_E4M3_POS_CODES[hi] % 2 == 0))
    code = np.where(pick_hi, _E4M3_POS_CODES[hi], _E4M3_POS_CODES[lo]).astype(np.uint8)
    code = np.where(np.isnan(y), np.uint8(0x7F), code)
    return code | sign


def append_kv(k_pages, v_pages, block_table, seq_lens, k_new, v_new):
    """Pools after each row's newest token is written to its tail page: row b's
    ``k_new[b], v_new[b]`` ([Hkv, 128]) go to token position ``seq_lens[b] - 1``, i.e. page
    ``block_table[b, pos // ps]``, slot ``pos % ps`` of the [pages, Hkv, ps, 128] pools.
    Rows with no tokens, or whose position falls outside the table or whose page falls
    outside the pool, are left alone.  (The reference's harness grows lengths without
    writing K/V, benchmark_serving_trace.py:285-298; this is the write a serving loop
    makes before the decode step.)  Returns new CPU tensors."""
    k_out, v_out = _cpu(k_pages).clone(), _cpu(v_pages).clone()
    table = _cpu(block_table)
    ps, pages = k_out.shape[2], k_out.shape[0]
    for b, length in enumerate(_cpu(seq_lens).tolist()):
        pos = int(length) - 1
        if pos < 0 or pos // ps >= table.shape[1]:
            continue
        page = int(table[b, pos // ps])
        if 0 <= page < pages:
            k_out[page, :, pos % ps] = _cpu(k_new)[b].to(k_out.dtype)
            v_out[page, :, pos % ps] = _cpu(v_new)[b].to(v_out.dtype)
    return k_out, v_out


def workqueue_decode(q_source, k_pages, v_pages, block_table, seq_lens, work_items,
                     split_offsets, q_indices, out_indices, out_rows, total_slots=None):
    """Result of the work-queue op for any work queue, float32 ``[out_rows, Hq, 128]``.

    Restates the reference's two kernels over a caller's queue, not only the builder's:
    - each item ``(row, kvh, split, tb, te)`` writes the partial state of its tile range
      for the G query heads of KV head ``kvh`` into slot ``split_offsets[row] + split``
      (cuh:294-363, :615-632).  A negative ``tb`` or ``te`` means the row-local split
      bound ``T*split//S`` or ``T*(split+1)//S`` (cuh:330-337, S = the row's slot count);
      tokens at or past ``seq_lens[row]`` are masked (cuh:217-219), so a range past the
      row's tiles contributes nothing, and a range with ``te <= tb`` is the neutral state
      (cuh:340-363);
    - row ``b``'s output folds every slot of ``[split_offsets[b], split_offsets[b+1])``
      (cuh:753-784) into output row ``out_indices[b]``.
    A slot that no item writes holds uninitialised memory in the reference (its result is
    then undefined); here it is the neutral state, which is what the builder's queues
    (empty splits emit no item) need.  Items whose row, KV head, split or slot lie outside
    their ranges are ignored (the reference writes out of bounds there).  When several
    items write one slot (a race in the reference), the last in queue order is kept.
    """
    q_source = _cpu(q_source)
    hq = q_source.shape[1]
    hkv = _cpu(k_pages).shape[1]
    g = hq // hkv
    table = _cpu(block_table)
    lens = [int(x) for x in _cpu(seq_lens).tolist()]
    offsets = [int(x) for x in _cpu(split_offsets).tolist()]
    items = [[int(x) for x in it] for it in _cpu(work_items).reshape(-1, 5).tolist()]
    q_idx = [int(x) for x in _cpu(q_indices).tolist()]
    o_idx = [int(x) for x in _cpu(out_indices).tolist()]
    batch = len(lens)
    slots = total_slots if total_slots is not None else offsets[-1]
    states = {}  # (slot, qh) -> (m, l, acc)
    rows = {}
    for row, kvh, split, tb, te in items:
        if not (0 <= row < batch and 0 <= kvh < hkv):
            continue
        n_split = offsets[row + 1] - offsets[row]
        slot = offsets[row] + split
        if not (0 <= split < n_split and 0 <= slot < slots):
            continue
        length = lens[row]
        total = (length + TILE - 1) // TILE
        tb = tb if tb >= 0 else total * split // n_split
        te = te if te >= 0 else total * (split + 1) // n_split
        if row not in rows:
            rows[row] = gather_row(k_pages, v_pages, table[row], length)
        k, v = rows[row]
        heads = range(kvh * g, (kvh + 1) * g)
        m, l, acc = split_partials(q_source[q_idx[row]], k, v, [(max(tb, 0), max(te, 0))])
        for h in heads:
            states[(slot, h)] = (m[h, 0], l[h, 0], acc[h, 0])
    out = torch.zeros(out_rows, hq, HEAD_DIM, dtype=torch.float32)
    neutral = (float(NEG_FLT_MAX), 0.0, np.zeros(HEAD_DIM))
    for b in range(batch):
        lo, hi = max(offsets[b], 0), min(offsets[b + 1], slots)
        if not 0 <= o_idx[b] < out_rows:
            continue
        for h in range(hq):
            picked = [states.get((s, h), neutral) for s in range(lo, hi)]
            if not picked:
                continue
            m = np.array([p[0] for p in picked])
            l = np.array([p[1] for p in picked])
            acc = np.stack([p[2] for p in picked])
            out[o_idx[b], h] = torch.from_numpy(lse_merge(m, l, acc)).float()
    return out
