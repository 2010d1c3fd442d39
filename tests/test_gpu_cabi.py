"""Parity through the bare C ABI (libpkv.so via ctypes), without the torch extension.

Binds the entry points with the ctypes argument lists a non-torch caller uses, and checks
the work-queue and grid ops against the repack + fp32 SDPA oracle (max-abs 2e-3, mean-abs
3e-4) and that an inconsistent argument returns PKV_ERR_INVALID_ARGUMENT with a message
instead of launching.
"""
import ctypes

import numpy as np
import pytest
import torch

import pkv_native
from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
P, I, Z = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t


@pytest.fixture(scope="module")
def lib(gpu):
    so = pkv_native.lib()
    so.pkv_paged_attention_workqueue.argtypes = [P, I, P, P, P, P, P, I, P, P, P, P, P, I, P, Z] + [I] * 11 + [P]
    so.pkv_paged_attention_workqueue.restype = ctypes.c_int
    so.pkv_paged_attention.argtypes = [P, P, P, P, P, P, Z] + [I] * 10 + [P]
    so.pkv_paged_attention.restype = ctypes.c_int
    return so


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_workqueue_through_c_abi(lib, gpu, dtype):
    lengths, rids = [40, 700, 1500, 33], [2, 0, 3, 1]
    hq, hkv, ps = 32, 8, 16
    case = make_case(lengths, hq, hkv, ps, dtype, seed=5, q_rows=4)
    meta = pkv_native.build_workqueue(lengths, rids, case.page_lists, ps, 6, False, hkv=hkv)
    dev = gpu
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    bt, sl, wi, so, qi, oi = (t(meta[k]) for k in ("block_table", "seq_lens", "work_items",
                                                   "split_offsets", "q_indices", "out_indices"))
    q, kp, vp = case.q.to(dev), case.k_pages.to(dev), case.v_pages.to(dev)
    counters = torch.zeros(len(lengths), hkv, dtype=torch.int32, device=dev)
    slots = meta["total_partial_slots"]
    ws = torch.empty(slots * hq * 130, dtype=torch.float32, device=dev)
    out = torch.full((len(lengths), hq, 128), float("nan"), dtype=dtype, device=dev)
    st = lib.pkv_paged_attention_workqueue(
        q.data_ptr(), q.size(0), kp.data_ptr(), vp.data_ptr(), bt.data_ptr(), sl.data_ptr(),
        wi.data_ptr(), wi.size(0), so.data_ptr(), counters.data_ptr(), qi.data_ptr(),
        oi.data_ptr(), out.data_ptr(), out.size(0), ws.data_ptr(), ws.numel() * 4,
        bt.size(0), hq, hkv, 128, kp.size(0), ps, bt.size(1), meta["bucket_length"], slots, 0,
        1 if dtype == torch.bfloat16 else 0, torch.cuda.current_stream().cuda_stream)
    assert st == 0, pkv_native.last_error()
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, meta["block_table"],
                              meta["seq_lens"], meta["q_indices"], meta["out_indices"])
    assert_parity(out, ref)


def test_grid_op_through_c_abi_and_invalid_argument(lib, gpu):
    hq, hkv, ps, ctx, splits = 32, 8, 16, 1000, 4
    case = make_case([ctx, ctx], hq, hkv, ps, torch.float16, seed=11)
    q, kp, vp, bt = (x.to(gpu) for x in (case.q, case.k_pages, case.v_pages, case.block_table))
    out = torch.full((2, hq, 128), float("nan"), dtype=torch.float16, device=gpu)
    ws = torch.empty(2 * hq * splits * 130, dtype=torch.float32, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    args = [q.data_ptr(), kp.data_ptr(), vp.data_ptr(), bt.data_ptr(), out.data_ptr(),
            ws.data_ptr(), ws.numel() * 4, 2, hq, hkv, 128, kp.size(0), ps, bt.size(1), ctx,
            splits, 0, stream]
    assert lib.pkv_paged_attention(*args) == 0, pkv_native.last_error()
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(out, ref)
    bad = list(args)
    bad[6] = 16  # workspace smaller than B * Hq * S * 130 floats
    sentinel = out.clone()
    assert lib.pkv_paged_attention(*bad) == 3
    assert "workspace" in pkv_native.last_error()
    bad = list(args)
    bad[9] = 7   # Hq not a multiple of Hkv
    assert lib.pkv_paged_attention(*bad) == 1
    torch.cuda.synchronize()
    assert torch.equal(out, sentinel)
