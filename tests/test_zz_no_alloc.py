"""pkv_paged_attention_workqueue_noalloc (static scratch, no workspace argument) through the
C ABI against pkv_paged_attention_workqueue with a caller workspace: identical outputs, bit
for bit, on two calls in a row (the second with a smaller input), for the two-launch and
the fused merge, and for the balanced schedule; and a request beyond the 16 MiB scratch
is rejected before any launch."""
import ctypes

import pytest
import torch

import pkv_native
from paged_cases import make_case

pytestmark = pytest.mark.gpu

_V, _I = ctypes.c_void_p, ctypes.c_int32
_QUEUE = [_V, _I, _V, _V, _V, _V, _V, _I, _V, _V, _V, _V, _V, _I]
_GEOM = [_I] * 11 + [_V]   # batch .. fused_merge, dtype, stream


@pytest.fixture(scope="module")
def lib(gpu):
    so = pkv_native.lib()
    so.pkv_paged_attention_workqueue.argtypes = _QUEUE + [_V, ctypes.c_size_t] + _GEOM
    so.pkv_paged_attention_workqueue.restype = ctypes.c_int
    so.pkv_paged_attention_workqueue_noalloc.argtypes = _QUEUE + _GEOM
    so.pkv_paged_attention_workqueue_noalloc.restype = ctypes.c_int
    return so


def _call(lib, case, lengths, hkv, splits, fused, gpu, workspace):
    hq = case.q.shape[1]
    meta = pkv_native.build_workqueue(lengths, list(range(len(lengths))), case.page_lists, 16,
                                      splits, False, hkv)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    bt, sl, wi, so, qi, oi = (t(meta[x]) for x in ("block_table", "seq_lens", "work_items",
                                                   "split_offsets", "q_indices", "out_indices"))
    b = len(lengths)
    counters = torch.zeros(b, hkv, dtype=torch.int32, device=gpu)
    out = torch.full((b, hq, 128), float("nan"), dtype=torch.float16, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    head = [q.data_ptr(), q.shape[0], k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(),
            wi.data_ptr(), wi.shape[0], so.data_ptr(), counters.data_ptr(), qi.data_ptr(),
            oi.data_ptr(), out.data_ptr(), b]
    tail = [b, hq, hkv, 128, k.shape[0], 16, bt.shape[1], meta["bucket_length"],
            meta["total_partial_slots"], int(fused), 0, stream]
    if workspace:
        ws = torch.empty(meta["total_partial_slots"] * hq * 130, dtype=torch.float32, device=gpu)
        st = lib.pkv_paged_attention_workqueue(*head, ws.data_ptr(), ws.numel() * 4, *tail)
    else:
        st = lib.pkv_paged_attention_workqueue_noalloc(*head, *tail)
    assert st == 0, pkv_native.last_error()
    torch.cuda.synchronize()
    assert torch.equal(counters, torch.zeros_like(counters))  # the fused merge resets them
    return out


@pytest.mark.parametrize("fused", [False, True])
def test_noalloc_equals_workspace_entry_on_two_calls(lib, gpu, fused):
    calls = [([3000, 40, 700, 1, 5000, 64], 8, 20, 3), ([300, 17], 4, 6, 4)]  # second smaller
    for lengths, hkv, splits, seed in calls:
        case = make_case(lengths, 32, hkv, 16, torch.float16, seed=seed)
        ref = _call(lib, case, lengths, hkv, splits, fused, gpu, workspace=True)
        got = _call(lib, case, lengths, hkv, splits, fused, gpu, workspace=False)
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref)


def test_noalloc_balanced_schedule_on_two_calls(lib, gpu):
    """A C4-sized queue (8 rows x 8 KV heads, G = 4, 20 splits: 2.66 MB of reference-sized
    states, which hold the balanced schedule's states, plan entries and check flags) takes
    the balanced schedule in the static scratch too; then a smaller one."""
    calls = [([20000, 300, 700, 1, 5000, 64, 31000, 513], 8, 20, 5), ([900, 4000], 8, 3, 6)]
    for i, (lengths, hkv, splits, seed) in enumerate(calls):
        meta = pkv_native.build_workqueue(lengths, list(range(len(lengths))),
                                          [[0]] * len(lengths), 16, splits, False, hkv)
        ws_bytes = meta["total_partial_slots"] * 32 * 130 * 4
        assert pkv_native.workqueue_schedule(len(lengths), 32, hkv, 16, ws_bytes) == (1 if i == 0 else 0)
        case = make_case(lengths, 32, hkv, 16, torch.float16, seed=seed)
        ref = _call(lib, case, lengths, hkv, splits, False, gpu, workspace=True)
        got = _call(lib, case, lengths, hkv, splits, False, gpu, workspace=False)
        assert torch.isfinite(got).all()
        assert torch.equal(got, ref)


def test_noalloc_rejects_more_than_the_static_scratch(lib, gpu):
    # 1009 slots x 32 heads x 130 floats > 16 MiB: rejected before anything is launched.
    case = make_case([64], 32, 8, 16, torch.float16, seed=1)
    meta = pkv_native.build_workqueue([64], [0], case.page_lists, 16, 2, False, 8)
    t = lambda a: torch.as_tensor(a, dtype=torch.int32, device=gpu)
    q, k, v = case.q.to(gpu), case.k_pages.to(gpu), case.v_pages.to(gpu)
    bt, sl, wi, so = (t(meta[x]) for x in ("block_table", "seq_lens", "work_items", "split_offsets"))
    idx = t([0])
    out = torch.zeros(1, 32, 128, dtype=torch.float16, device=gpu)
    st = lib.pkv_paged_attention_workqueue_noalloc(
        q.data_ptr(), 1, k.data_ptr(), v.data_ptr(), bt.data_ptr(), sl.data_ptr(), wi.data_ptr(),
        wi.shape[0], so.data_ptr(), None, idx.data_ptr(), idx.data_ptr(), out.data_ptr(), 1,
        1, 32, 8, 128, k.shape[0], 16, bt.shape[1], 64, 1009, 0, 0,
        torch.cuda.current_stream().cuda_stream)
    assert st == 3 and "static scratch" in pkv_native.last_error()
    torch.cuda.synchronize()
    assert torch.equal(out, torch.zeros_like(out))
