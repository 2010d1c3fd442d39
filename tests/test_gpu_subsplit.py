"""Split launches of few units cut into sub-splits (workspace of split_workspace_floats),
for the fp8 and fused-append variants of the grid ops: against the repack + fp32 SDPA
oracle, against the same op with the reference's workspace size (the caller's split
only; same output to fp32 rounding), and for the append variants bit for bit against
append_kv followed by the op with the same workspace."""
import pytest
import torch

from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16, BF16, F8 = torch.float16, torch.bfloat16, torch.float8_e4m3fn


def _quantise(x, scale):
    return (x.float() / scale).clamp(-448.0, 448.0).to(F8)


@pytest.mark.parametrize("dtype", [F16, BF16])
def test_indexed_fp8_subdivided(ext, gpu, dtype):
    lengths, hq, hkv, splits, ks, vs = [6000, 40], 32, 8, 4, 0.03, 0.02  # 64 units
    case = make_case(lengths, hq, hkv, 16, dtype, seed=31)
    k8, v8 = _quantise(case.k_pages, ks).to(gpu), _quantise(case.v_pages, vs).to(gpu)
    b, ctx = len(lengths), max(lengths)
    full = ext.split_workspace_floats(b, hq, hkv, ctx, splits)
    ref_floats = b * hq * splits * 130
    assert full >= 2 * ref_floats
    idx = torch.tensor([1, 0], dtype=torch.int32, device=gpu)
    outs = []
    for floats in (full, ref_floats):
        out = torch.full((b, hq, 128), float("nan"), dtype=dtype, device=gpu)
        ws = torch.empty(floats, dtype=torch.float32, device=gpu)
        ext.paged_attention_indexed_fp8(case.q.to(gpu), k8, v8, case.block_table.to(gpu),
                                        case.seq_lens.to(gpu), idx, idx, out, ws, ctx, 16,
                                        splits, ks, vs)
        torch.cuda.synchronize()
        outs.append(out)
    ref = oracle.paged_decode(case.q, oracle.dequantize_e4m3(k8.cpu(), ks),
                              oracle.dequantize_e4m3(v8.cpu(), vs), case.block_table,
                              case.seq_lens, idx.cpu(), idx.cpu(), b)
    for out in outs:
        assert_parity(out, ref)
    assert (outs[0].float() - outs[1].float()).abs().max().item() < 1e-3


@pytest.mark.parametrize("op", ["indexed", "masked"])
def test_append_subdivided(ext, gpu, op):
    lengths, hq, hkv, splits = [5000, 700, 33], 32, 8, 4  # 96 units
    b, ctx = len(lengths), max(lengths)
    case = make_case(lengths, hq, hkv, 16, F16, seed=41)
    gen = torch.Generator().manual_seed(5)
    kn = torch.randn(b, hkv, 128, generator=gen).half().to(gpu)
    vn = torch.randn(b, hkv, 128, generator=gen).half().to(gpu)
    bt, sl, q = case.block_table.to(gpu), case.seq_lens.to(gpu), case.q.to(gpu)
    idx = torch.arange(b, dtype=torch.int32, device=gpu)
    full = ext.split_workspace_floats(b, hq, hkv, ctx, splits)
    assert full >= 2 * b * hq * splits * 130
    ws = torch.empty(full, dtype=torch.float32, device=gpu)

    def run(fused):
        k, v = case.k_pages.to(gpu), case.v_pages.to(gpu)
        out = torch.full((b, hq, 128), float("nan"), dtype=F16, device=gpu)
        if not fused:
            ext.append_kv(kn, vn, k, v, bt, sl)
        if op == "indexed":
            args = (q, k, v, bt, sl, idx, idx, out, ws, ctx, 16, splits)
            (ext.paged_attention_indexed_append(*args, kn, vn) if fused
             else ext.paged_attention_indexed(*args))
        else:
            args = (q, k, v, bt, sl, out, ws, ctx, 16, splits)
            (ext.paged_attention_masked_append(*args, kn, vn) if fused
             else ext.paged_attention_masked(*args))
        torch.cuda.synchronize()
        return out, k, v

    (o1, k1, v1), (o2, k2, v2) = run(False), run(True)
    assert torch.equal(k2, k1) and torch.equal(v2, v1)
    assert torch.equal(o2, o1)
    k_ref, v_ref = oracle.append_kv(case.k_pages, case.v_pages, case.block_table, case.seq_lens,
                                    kn.cpu(), vn.cpu())
    ref = oracle.paged_decode(case.q, k_ref, v_ref, case.block_table, case.seq_lens)
    assert_parity(o2, ref)
