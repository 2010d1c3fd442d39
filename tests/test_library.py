"""The C-ABI library and the op module load and validate on the CPU (no GPU work).

* libpkv.so exports every function include/pkv.h declares.
* The op module exposes the reference's four op names (plus the two stage ops).
* Argument checks reject bad input before any device work: through the op surface
  (the reference's TORCH_CHECK messages, tests/persistentkv_torch_extension.cu:9-31) and
  through the C ABI (status codes instead of the reference's process exit).
"""
import ctypes

import pytest
import torch

import pkv_native


def test_library_exports_every_header_function():
    lib = pkv_native.lib()
    names = pkv_native.header_functions()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_op_module_surface():
    import persistentkv_torch_ext as ext
    for name in ("paged_attention", "paged_attention_masked", "paged_attention_indexed",
                 "paged_attention_workqueue", "workqueue_decode", "workqueue_merge"):
        assert callable(getattr(ext, name))


def test_op_rejects_cpu_tensors_with_reference_messages():
    import persistentkv_torch_ext as ext
    q = torch.zeros(1, 32, 128, dtype=torch.float16)
    k = torch.zeros(4, 8, 16, 128, dtype=torch.float16)
    bt = torch.zeros(1, 4, dtype=torch.int32)
    out = torch.zeros(1, 32, 128, dtype=torch.float16)
    ws = torch.zeros(0)
    with pytest.raises(RuntimeError, match="q must be a CUDA tensor"):
        ext.paged_attention(q, k, k, bt, out, ws, 64, 16, 1)
    with pytest.raises(RuntimeError, match="q has wrong dtype"):
        ext.paged_attention(q.float(), k, k, bt, out, ws, 64, 16, 1)
    with pytest.raises(RuntimeError, match="q_source must be a CUDA tensor"):
        ext.paged_attention_indexed(q, k, k, bt, bt[0], bt[0, :1], bt[0, :1], out, ws, 64, 16, 1)


def test_workspace_sizes():
    lib = pkv_native.lib()
    assert lib.pkv_workspace_bytes(8, 32, 1) == 0                      # cuh:894-895
    assert lib.pkv_workspace_bytes(8, 32, 20) == 8 * 32 * 20 * 130 * 4  # cuh:896-897
    assert lib.pkv_workqueue_workspace_bytes(160, 32) == 160 * 32 * 130 * 4
    # direct launches: ~256 units of >= 2 tiles from the caller's workspace
    assert pkv_native.direct_workspace_bytes(1, 32, 8, 2048) == 1 * 32 * 32 * 130 * 4
    assert pkv_native.direct_workspace_bytes(1, 32, 8, 200) == 1 * 32 * 3 * 130 * 4  # 7 tiles
    assert pkv_native.direct_workspace_bytes(1, 32, 8, 64) == 0    # 2 tiles: not split
    assert pkv_native.direct_workspace_bytes(16, 32, 8, 8192) == 0  # 128 units: not split
    # split launches of few units: sub-splits to about one unit per CU (256 without a GPU)
    ref = lambda b, hq, s: lib.pkv_workspace_bytes(b, hq, s)
    assert pkv_native.split_workspace_bytes(1, 32, 8, 8192, 16) == ref(1, 32, 32)   # 128 units, k 2
    assert pkv_native.split_workspace_bytes(1, 8, 8, 8192, 4) == ref(1, 8, 32)      # 32 units, k 8
    assert pkv_native.split_workspace_bytes(1, 32, 8, 32768, 32) == ref(1, 32, 32)  # 256 units
    assert pkv_native.split_workspace_bytes(1, 32, 8, 1024, 16) == ref(1, 32, 16)   # 32 tiles only
    assert pkv_native.split_workspace_bytes(8, 32, 32, 4096, 8) == ref(8, 32, 8)    # 2048 units
    assert pkv_native.split_workspace_bytes(1, 32, 8, 8192, 1) == 0                 # direct launch
    # the balanced work-queue schedule: (B*Hkv + 4 waves x CUs) groups of G states, the
    # state count rounded up to even (acc 16-byte aligned), then one 16-byte plan entry per
    # pair, then one queue-check flag per decode workgroup (one per CU)
    assert pkv_native.workqueue_balanced_workspace_bytes(8, 32, 8) == (8 * 8 + 4 * 256) * 4 * 520 + 8 * 8 * 16 + 256 * 4
    assert pkv_native.workqueue_balanced_workspace_bytes(3, 3, 1) == ((3 + 4 * 256) * 3 + 1) * 520 + 3 * 16 + 256 * 4
    assert pkv_native.workqueue_balanced_workspace_bytes(8, 32, 1) == 0    # G = 32: never taken
    assert pkv_native.workqueue_balanced_workspace_bytes(257, 32, 8) == 0  # more than 256 rows


def _call_paged(**overrides):
    lib = pkv_native.lib()
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    args = dict(q=fake, k=fake, v=fake, table=fake, out=fake, ws=None, ws_bytes=0, batch=1, hq=32,
                hkv=8, d=128, pages=16, ps=16, maxp=4, ctx=64, splits=1, dtype=0)
    args.update(overrides)
    f = lib.pkv_paged_attention
    f.restype = ctypes.c_int
    return f(args["q"], args["k"], args["v"], args["table"], args["out"], args["ws"],
             ctypes.c_size_t(args["ws_bytes"]), args["batch"], args["hq"], args["hkv"], args["d"],
             args["pages"], args["ps"], args["maxp"], args["ctx"], args["splits"], args["dtype"],
             None)


@pytest.mark.parametrize("overrides,status,text", [
    (dict(d=64), 2, "d=128"),
    (dict(hq=30), 1, "divisible"),
    (dict(hq=264, hkv=8), 2, "G=Hq/Hkv"),
    (dict(splits=3), 1, "num_splits=3 exceeds"),
    (dict(ctx=128), 1, "block_table has 4 pages"),
    (dict(splits=2), 3, "workspace"),
    (dict(dtype=7), 2, "dtype"),
    (dict(ps=0), 1, "page_size"),
])
def test_c_abi_status_codes(overrides, status, text):
    st = _call_paged(**overrides)
    assert st == status
    assert text in pkv_native.last_error()


def test_c_abi_empty_batch_is_a_no_op():
    assert _call_paged(batch=0) == 0
