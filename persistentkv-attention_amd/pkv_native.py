"""ctypes bindings of the PersistentKV C ABI (include/pkv.h) in ``libpkv.so``.

Exposes the host scheduling entry points (split policy, cost-model router and the
compact work-queue builder) to Python with numpy arrays, and the raw library handle for
callers that drive the device entry points directly.  ``torch`` is imported first when
available so that the library binds to torch's HIP runtime rather than loading a second
copy.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

try:  # bind to torch's HIP runtime when torch is present
    import torch  # noqa: F401
except ImportError:  # pragma: no cover - torch is part of the supported environment
    torch = None

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "libpkv.so")
HEADER_PATH = os.path.join(os.path.dirname(_HERE), "include", "pkv.h")

POLICY_REFERENCE = 0
POLICY_MI355X = 1
ROUTES = {0: "flashinfer", 1: "persistentkv_bucket", 2: "persistentkv_workqueue"}
ROUTE_IDS = {v: k for k, v in ROUTES.items()}

PKV_OK = 0
PKV_ERR_CAPACITY = 5


class CostModel(ctypes.Structure):
    _fields_ = [
        ("num_q_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("compute_units", ctypes.c_int32),
        ("read_gbps", ctypes.c_double),
        ("launch_overhead_us", ctypes.c_double),
        ("min_ctas_per_cu", ctypes.c_double),
        ("supported_group", ctypes.c_int32),
        ("min_long_context", ctypes.c_int32),
        ("policy", ctypes.c_int32),
        ("unit_round_us", ctypes.c_double),
        ("grid_merge_us", ctypes.c_double),
        ("queue_merge_us", ctypes.c_double),
    ]


_I32 = ctypes.c_int32
_PI32 = ctypes.POINTER(ctypes.c_int32)
_lib = None


def lib():
    """The loaded ``libpkv.so`` with argument types declared."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY_PATH):
        raise ImportError(f"{LIBRARY_PATH} is not built; run `make -C persistentkv-attention_amd/csrc`")
    so = ctypes.CDLL(LIBRARY_PATH)
    so.pkv_last_error.restype = ctypes.c_char_p
    so.pkv_status_string.restype = ctypes.c_char_p
    so.pkv_status_string.argtypes = [ctypes.c_int]
    so.pkv_workspace_bytes.restype = ctypes.c_size_t
    so.pkv_workspace_bytes.argtypes = [_I32, _I32, _I32]
    so.pkv_workqueue_workspace_bytes.restype = ctypes.c_size_t
    so.pkv_workqueue_workspace_bytes.argtypes = [_I32, _I32]
    so.pkv_direct_workspace_bytes.restype = ctypes.c_size_t
    so.pkv_direct_workspace_bytes.argtypes = [_I32, _I32, _I32, _I32]
    so.pkv_split_workspace_bytes.restype = ctypes.c_size_t
    so.pkv_split_workspace_bytes.argtypes = [_I32, _I32, _I32, _I32, _I32]
    so.pkv_workqueue_balanced_workspace_bytes.restype = ctypes.c_size_t
    so.pkv_workqueue_balanced_workspace_bytes.argtypes = [_I32, _I32, _I32]
    so.pkv_workqueue_schedule.restype = ctypes.c_int
    so.pkv_workqueue_schedule.argtypes = [_I32, _I32, _I32, _I32, ctypes.c_size_t, _I32]
    so.pkv_cost_model_preset.argtypes = [_I32, ctypes.POINTER(CostModel)]
    so.pkv_cost_model_preset.restype = None
    so.pkv_choose_workqueue_row_splits.argtypes = [_I32] * 6
    so.pkv_choose_workqueue_row_splits.restype = _I32
    so.pkv_choose_splits.argtypes = [_PI32] + [_I32] * 6
    so.pkv_choose_splits.restype = _I32
    so.pkv_model_bucket_splits.argtypes = [_PI32, _I32, _I32, _I32]
    so.pkv_model_bucket_splits.restype = _I32
    so.pkv_model_workqueue_splits.argtypes = [_PI32, _I32, _I32, _I32]
    so.pkv_model_workqueue_splits.restype = _I32
    so.pkv_estimate_route_ms.argtypes = [_PI32, _I32, _I32, _I32, ctypes.POINTER(CostModel)]
    so.pkv_estimate_route_ms.restype = ctypes.c_double
    so.pkv_choose_adaptive_route.argtypes = [_PI32, _I32, ctypes.POINTER(CostModel), _PI32,
                                             ctypes.POINTER(ctypes.c_double)]
    so.pkv_choose_adaptive_route.restype = _I32
    so.pkv_workqueue_size.argtypes = [_PI32, _I32, _I32, _I32, _I32, _I32, _I32, _PI32, _PI32]
    so.pkv_workqueue_size.restype = ctypes.c_int
    so.pkv_build_workqueue.argtypes = [
        _PI32, _PI32, _I32, _PI32, _PI32, _I32, _I32, _I32, _I32, _I32, _I32,
        _PI32, _I32, _PI32, _PI32, _PI32, _PI32, _PI32, _I32, _PI32, _PI32, _PI32]
    so.pkv_build_workqueue.restype = ctypes.c_int
    so.pkv_round_bucket_length.argtypes = [_I32] * 4
    so.pkv_round_bucket_length.restype = _I32
    so.pkv_use_single_bucket.argtypes = [_PI32, _I32, _I32, _I32]
    so.pkv_use_single_bucket.restype = _I32
    _PI64 = ctypes.POINTER(ctypes.c_int64)
    so.pkv_build_buckets.argtypes = [
        _PI32, _PI32, _I32, _PI32, _PI32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32,
        _PI32, _PI32, _PI32, _PI32, _PI32, _PI32, _PI32, _PI32, _PI32, ctypes.c_int64, _PI64]
    so.pkv_build_buckets.restype = ctypes.c_int
    _lib = so
    return so


def last_error() -> str:
    return lib().pkv_last_error().decode()


def direct_workspace_bytes(batch, hq, hkv, context) -> int:
    """Workspace bytes with which a direct (num_splits == 1) launch runs its full internal
    split (pkv_direct_workspace_bytes)."""
    return int(lib().pkv_direct_workspace_bytes(batch, hq, hkv, context))


def split_workspace_bytes(batch, hq, hkv, context, num_splits) -> int:
    """Workspace bytes with which a split launch of few units runs its full internal
    sub-split (pkv_split_workspace_bytes); the reference's size when it is not sub-split."""
    return int(lib().pkv_split_workspace_bytes(batch, hq, hkv, context, num_splits))


def workqueue_balanced_workspace_bytes(batch, hq, hkv) -> int:
    """Workspace bytes with which the work-queue op takes its balanced schedule on the
    current device (pkv_workqueue_balanced_workspace_bytes)."""
    return int(lib().pkv_workqueue_balanced_workspace_bytes(batch, hq, hkv))


def workqueue_schedule(batch, hq, hkv, page_size, workspace_bytes, fused_merge=False) -> int:
    """1 when the work-queue op takes the balanced schedule, else 0 (pkv_workqueue_schedule)."""
    return int(lib().pkv_workqueue_schedule(batch, hq, hkv, page_size, workspace_bytes,
                                            int(bool(fused_merge))))


def _arr(values):
    a = np.ascontiguousarray(np.asarray(values, dtype=np.int32))
    return a, a.ctypes.data_as(_PI32)


def cost_model(policy: int = POLICY_REFERENCE, **overrides) -> CostModel:
    m = CostModel()
    lib().pkv_cost_model_preset(policy, ctypes.byref(m))
    for key, value in overrides.items():
        setattr(m, key, value)
    return m


def choose_workqueue_row_splits(length, active_count, requested_splits, auto_splits,
                                hkv=8, policy=POLICY_REFERENCE) -> int:
    return lib().pkv_choose_workqueue_row_splits(length, active_count, requested_splits,
                                                 int(bool(auto_splits)), hkv, policy)


def choose_splits(lengths, requested_splits, auto_splits, single_bucket, hkv=8,
                  policy=POLICY_REFERENCE) -> int:
    a, p = _arr(lengths)
    return lib().pkv_choose_splits(p, len(a), requested_splits, int(bool(auto_splits)),
                                   int(bool(single_bucket)), hkv, policy)


def model_bucket_splits(lengths, hkv=8, policy=POLICY_REFERENCE) -> int:
    a, p = _arr(lengths)
    return lib().pkv_model_bucket_splits(p, len(a), hkv, policy)


def model_workqueue_splits(lengths, hkv=8, policy=POLICY_REFERENCE) -> int:
    a, p = _arr(lengths)
    return lib().pkv_model_workqueue_splits(p, len(a), hkv, policy)


def estimate_route_ms(lengths, route, splits, model: CostModel | None = None) -> float:
    a, p = _arr(lengths)
    m = model or cost_model()
    return lib().pkv_estimate_route_ms(p, len(a), ROUTE_IDS[route], splits, ctypes.byref(m))


def choose_adaptive_route(lengths, model: CostModel | None = None):
    """``(route_name, splits, estimated_ms)`` for one decode step."""
    a, p = _arr(lengths)
    m = model or cost_model()
    splits = ctypes.c_int32()
    ms = ctypes.c_double()
    route = lib().pkv_choose_adaptive_route(p, len(a), ctypes.byref(m), ctypes.byref(splits),
                                            ctypes.byref(ms))
    return ROUTES[route], splits.value, ms.value


def build_workqueue(lengths, request_ids, page_lists, page_size, requested_splits, auto_splits,
                    hkv=8, policy=POLICY_REFERENCE, hq=32):
    """One step's work-queue metadata as numpy int32 arrays (see pkv_build_workqueue).
    ``hq`` (query heads) only steers the MI355X policy's item size."""
    count = len(lengths)
    la, lp = _arr(lengths)
    ra, rp = _arr(request_ids)
    indptr = np.zeros(count + 1, dtype=np.int32)
    for r, pages in enumerate(page_lists):
        indptr[r + 1] = indptr[r] + len(pages)
    ids = np.ascontiguousarray(np.concatenate([np.asarray(p, dtype=np.int32) for p in page_lists])
                               if count else np.zeros(0, dtype=np.int32))
    tasks, slots = _I32(), _I32()
    st = lib().pkv_workqueue_size(lp, count, requested_splits, int(bool(auto_splits)), hq, hkv,
                                  policy, ctypes.byref(tasks), ctypes.byref(slots))
    if st != PKV_OK:
        raise ValueError(f"pkv_workqueue_size failed with status {st}")
    bucket = int(la.max()) if count else 0
    cols = -(-bucket // page_size) if bucket > 0 else 0
    table = np.zeros((count, max(cols, 1)), dtype=np.int32)
    seq = np.zeros(count, dtype=np.int32)
    qi = np.zeros(count, dtype=np.int32)
    oi = np.zeros(count, dtype=np.int32)
    items = np.zeros((max(tasks.value, 1), 5), dtype=np.int32)
    offs = np.zeros(count + 1, dtype=np.int32)
    out_cols, out_tasks, out_slots = _I32(), _I32(), _I32()
    st = lib().pkv_build_workqueue(
        lp, rp, count, indptr.ctypes.data_as(_PI32), ids.ctypes.data_as(_PI32), page_size,
        requested_splits, int(bool(auto_splits)), hq, hkv, policy, table.ctypes.data_as(_PI32),
        table.size, ctypes.byref(out_cols), seq.ctypes.data_as(_PI32), qi.ctypes.data_as(_PI32),
        oi.ctypes.data_as(_PI32), items.ctypes.data_as(_PI32), items.shape[0],
        ctypes.byref(out_tasks), offs.ctypes.data_as(_PI32), ctypes.byref(out_slots))
    if st != PKV_OK:
        raise ValueError(f"pkv_build_workqueue failed with status {st}")
    row_splits = np.diff(offs)
    return dict(bucket_length=bucket, block_table=table[:, :out_cols.value], seq_lens=seq,
                q_indices=qi, out_indices=oi, work_items=items[:out_tasks.value],
                split_offsets=offs, total_partial_slots=int(out_slots.value),
                splits=int(max(1, row_splits.max())) if count else 1)


def round_bucket_length(length, bucket_tokens, allocated_pages, page_size=16) -> int:
    return lib().pkv_round_bucket_length(length, bucket_tokens, allocated_pages, page_size)


def use_single_bucket(lengths, requested_single_bucket, adaptive_route) -> bool:
    a, p = _arr(lengths)
    return bool(lib().pkv_use_single_bucket(p, len(a), int(bool(requested_single_bucket)),
                                            int(bool(adaptive_route))))


def build_buckets(lengths, request_ids, page_lists, page_size, requested_splits, auto_splits,
                  bucket_tokens=0, single_bucket=False, adaptive_route=False, hkv=8,
                  policy=POLICY_REFERENCE):
    """One step's length-bucket metadata (pkv_build_buckets): a list of dicts with
    bucket_length, block_table [rows, cols], seq_lens, q_indices, out_indices, splits."""
    count = len(lengths)
    la, lp = _arr(lengths)
    ra, rp = _arr(request_ids)
    indptr = np.zeros(count + 1, dtype=np.int32)
    for r, pages in enumerate(page_lists):
        indptr[r + 1] = indptr[r] + len(pages)
    ids = np.ascontiguousarray(np.concatenate([np.asarray(p, dtype=np.int32) for p in page_lists])
                               if count else np.zeros(0, dtype=np.int32))
    n_buckets, elems = _I32(), ctypes.c_int64()
    per = [np.zeros(max(count, 1), dtype=np.int32) for _ in range(7)]
    blen, brows, bsplit, bcols, seq, qi, oi = per
    args = lambda tables, cap: (
        lp, rp, count, indptr.ctypes.data_as(_PI32), ids.ctypes.data_as(_PI32), page_size,
        requested_splits, int(bool(auto_splits)), bucket_tokens, int(bool(single_bucket)),
        int(bool(adaptive_route)), hkv, policy, ctypes.byref(n_buckets),
        *(x.ctypes.data_as(_PI32) for x in per), tables, cap, ctypes.byref(elems))
    st = lib().pkv_build_buckets(*args(None, 0))
    if st not in (PKV_OK, PKV_ERR_CAPACITY):
        raise ValueError(f"pkv_build_buckets failed with status {st}")
    tables = np.zeros(max(int(elems.value), 1), dtype=np.int32)
    st = lib().pkv_build_buckets(*args(tables.ctypes.data_as(_PI32), tables.size))
    if st != PKV_OK:
        raise ValueError(f"pkv_build_buckets failed with status {st}")
    out, r0, t0 = [], 0, 0
    for j in range(n_buckets.value):
        n, c = int(brows[j]), int(bcols[j])
        out.append(dict(bucket_length=int(blen[j]), block_table=tables[t0:t0 + n * c].reshape(n, c),
                        seq_lens=seq[r0:r0 + n].copy(), q_indices=qi[r0:r0 + n].copy(),
                        out_indices=oi[r0:r0 + n].copy(), splits=int(bsplit[j])))
        r0 += n
        t0 += n * c
    return out


def header_functions(path: str = HEADER_PATH):
    """Names of the functions declared in include/pkv.h."""
    import re
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"\b([a-z_][a-z0-9_]*)\s*\(", text)
    return sorted({n for n in names if n.startswith("pkv_")})
