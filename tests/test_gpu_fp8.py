"""fp8 (OCP e4m3) K/V ops against the repack + fp32 SDPA oracle on the dequantised K/V.

K and V pages are quantised on the host with torch's float8_e4m3fn (round to nearest even,
after clamping to +-448) under per-tensor scales; the oracle attends to k_scale * e4m3(k8)
and v_scale * e4m3(v8), decoded by oracle.attention.dequantize_e4m3 from the format's
definition (pinned in tests/test_oracle_fp8.py).  The engine unpacks e4m3 exactly to
fp16 / bf16 in registers, so the comparison keeps the 2e-3 / 3e-4 gate of the 2-byte ops.  One case fills
a K and a V page with every finite e4m3 code (both signs, subnormals, +-448), which pins
the unpacking instruction's format and byte order: a misread code moves its token's
score or value.
"""
import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu

F16, BF16, F8 = torch.float16, torch.bfloat16, torch.float8_e4m3fn


def quantise(x, scale):
    return (x.float() / scale).clamp(-448.0, 448.0).to(F8)


def dequantise(x8, scale):
    return oracle.dequantize_e4m3(x8, scale)  # the closed-form decode, pinned on the CPU


def every_code_page(page_size, hkv, seed):
    """[hkv, page_size, 128] fp8 holding the 254 finite e4m3 codes (0x7f and 0xff are NaN),
    permuted per head and repeated to fill the page."""
    codes = torch.tensor([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=torch.uint8)
    gen = torch.Generator().manual_seed(seed)
    n = hkv * page_size * 128
    idx = torch.cat([torch.randperm(len(codes), generator=gen) for _ in range(-(-n // len(codes)))])
    return codes[idx[:n]].view(hkv, page_size, 128).view(F8)


def _run_queue_fp8(ext, gpu, case, k8, v8, meta, hq, hkv, ks, vs, fused):
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    b = len(meta["seq_lens"])
    out = torch.full((b, hq, 128), float("nan"), dtype=case.q.dtype, device=gpu)
    ws = torch.empty(meta["total_partial_slots"] * hq * 130, dtype=torch.float32, device=gpu)
    counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
    ext.paged_attention_workqueue_fp8(
        case.q.to(gpu), k8.to(gpu), v8.to(gpu), t(meta["block_table"]), t(meta["seq_lens"]),
        t(meta["work_items"]), t(meta["split_offsets"]), counters, t(meta["q_indices"]),
        t(meta["out_indices"]), out, ws, meta["bucket_length"], case.page_size,
        meta["total_partial_slots"], fused, ks, vs)
    torch.cuda.synchronize()
    return out, counters


# (lengths, Hq, Hkv, page_size, requested splits, dtype, k_scale, v_scale)
QUEUE = [
    ([300, 17000, 700, 256], 32, 8, 16, 20, F16, 0.02, 0.03),   # C4-like, G = 4
    ([2000, 4000, 900], 32, 1, 32, 12, BF16, 0.05, 0.01),       # G = 32, page 32
    ([1500, 77], 32, 4, 32, 6, BF16, 0.02, 0.02),               # G = 8
    ([5000, 120], 32, 32, 16, 8, F16, 0.01, 0.05),              # G = 1
]


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("lengths,hq,hkv,ps,req,dtype,ks,vs", QUEUE)
def test_workqueue_fp8(ext, gpu, lengths, hq, hkv, ps, req, dtype, ks, vs, fused):
    case = make_case(lengths, hq, hkv, ps, dtype, seed=len(lengths) + req, q_rows=len(lengths) + 2)
    k8, v8 = quantise(case.k_pages, ks), quantise(case.v_pages, vs)
    ids = [len(lengths) + 1 - i for i in range(len(lengths))]
    meta = pkv_native.build_workqueue(case.seq_lens.tolist(), ids, case.page_lists, ps, req,
                                      False, hkv)
    out, counters = _run_queue_fp8(ext, gpu, case, k8, v8, meta, hq, hkv, ks, vs, fused)
    ref = oracle.paged_decode(case.q, dequantise(k8, ks), dequantise(v8, vs), meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    assert_parity(out, ref)
    assert int(counters.abs().sum()) == 0


@pytest.mark.parametrize("dtype", [F16, BF16])
@pytest.mark.parametrize("splits", [1, 4])
def test_indexed_fp8(ext, gpu, splits, dtype):
    lengths = [400, 33, 1200]
    ks, vs = 0.03, 0.02
    case = make_case(lengths, 32, 8, 16, dtype, seed=11 + splits, q_rows=5)
    k8, v8 = quantise(case.k_pages, ks), quantise(case.v_pages, vs)
    q_idx = torch.tensor([4, 0, 2], dtype=torch.int32)
    o_idx = torch.tensor([3, 0, 5], dtype=torch.int32)
    out = torch.full((6, 32, 128), 7.0, dtype=dtype, device=gpu)
    ws = torch.empty(3 * 32 * splits * 130 if splits > 1 else 0, dtype=torch.float32, device=gpu)
    ext.paged_attention_indexed_fp8(case.q.to(gpu), k8.to(gpu), v8.to(gpu),
                                    case.block_table.to(gpu), case.seq_lens.to(gpu),
                                    q_idx.to(gpu), o_idx.to(gpu), out, ws, max(lengths), 16,
                                    splits, ks, vs)
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, dequantise(k8, ks), dequantise(v8, vs), case.block_table,
                              case.seq_lens, q_idx, o_idx, 6)
    assert_parity(out, ref)
    assert torch.all(out[[1, 2, 4]].float().cpu() == 7.0)


def test_every_e4m3_code(ext, gpu):
    """Pages of every finite code; scales keep the scores and outputs O(1)."""
    ps, hkv, hq, ks, vs = 16, 2, 8, 1.0 / 448.0, 1.0 / 128.0
    case = make_case([32, 20], hq, hkv, ps, F16, seed=5, table="contiguous")
    n_pages = case.k_pages.shape[0]
    k8 = torch.stack([every_code_page(ps, hkv, 100 + p) for p in range(n_pages)])
    v8 = torch.stack([every_code_page(ps, hkv, 200 + p) for p in range(n_pages)])
    meta = pkv_native.build_workqueue(case.seq_lens.tolist(), [0, 1], case.page_lists, ps, 2,
                                      False, hkv)
    out, _ = _run_queue_fp8(ext, gpu, case, k8, v8, meta, hq, hkv, ks, vs, False)
    ref = oracle.paged_decode(case.q, dequantise(k8, ks), dequantise(v8, vs), meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    assert_parity(out, ref)


def test_fp8_validation(ext, gpu):
    case = make_case([64], 32, 8, 8, F16)
    k8 = quantise(case.k_pages, 0.02).to(gpu)
    q, bt, sl = case.q.to(gpu), case.block_table.to(gpu), case.seq_lens.to(gpu)
    idx = torch.zeros(1, dtype=torch.int32, device=gpu)
    out = torch.empty(1, 32, 128, dtype=F16, device=gpu)
    empty = torch.empty(0, dtype=torch.float32, device=gpu)
    with pytest.raises(RuntimeError, match="multiple of 16"):
        ext.paged_attention_indexed_fp8(q, k8, k8, bt, sl, idx, idx, out, empty, 64, 8, 1, 1.0, 1.0)
    case16 = make_case([64], 32, 8, 16, F16)
    k16 = quantise(case16.k_pages, 0.02).to(gpu)
    bt16 = case16.block_table.to(gpu)
    with pytest.raises(RuntimeError, match="k_scale"):
        ext.paged_attention_indexed_fp8(q, k16, k16, bt16, sl, idx, idx, out, empty, 64, 16, 1,
                                        0.0, 1.0)
    with pytest.raises(RuntimeError, match="wrong dtype"):
        ext.paged_attention_indexed_fp8(q, case16.k_pages.to(gpu), case16.v_pages.to(gpu), bt16,
                                        sl, idx, idx, out, empty, 64, 16, 1, 1.0, 1.0)
