"""ctypes wrapper of oracle/pkv_oracle.c (test infrastructure only).

Loads ``oracle/_build/libpkv_oracle.so`` (built by ``make -C oracle`` or
``__graft_entry__.build()``).  See pkv_oracle.c for the reference lines each function
restates.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libpkv_oracle.so")
_lib = None

_F = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_I = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is not built; run `make -C oracle`")
        so = ctypes.CDLL(LIB_PATH)
        so.pkv_oracle_paged_decode.argtypes = [_F, _F, _F, _I, ctypes.c_int32, ctypes.c_int32,
                                               ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, _F]
        so.pkv_oracle_paged_decode.restype = None
        so.pkv_oracle_split_partial.argtypes = [_F, _F, _F, _I] + [ctypes.c_int32] * 6 + [
            ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float), _F]
        so.pkv_oracle_split_partial.restype = None
        so.pkv_oracle_lse_merge.argtypes = [_F, _F, _F, ctypes.c_int32, _F]
        so.pkv_oracle_lse_merge.restype = None
        so.pkv_oracle_cpu_gqa_attention.argtypes = [_F, _F, _F, _F] + [ctypes.c_int] * 5
        so.pkv_oracle_cpu_gqa_attention.restype = None
        so.pkv_oracle_smoke_case.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        so.pkv_oracle_smoke_inputs.argtypes = [ctypes.c_int, _F, _F, _F]
        _lib = so
    return _lib


def paged_decode_row(q_row, k_pool, v_pool, table_row, page_size, length, num_splits):
    """fp32 split + merge decode of one query row.  Pools are float32 numpy
    ``[pages, Hkv, page_size, 128]``; returns ``[Hq, 128]``."""
    q_row = np.ascontiguousarray(q_row, dtype=np.float32)
    k_pool = np.ascontiguousarray(k_pool, dtype=np.float32)
    v_pool = np.ascontiguousarray(v_pool, dtype=np.float32)
    table_row = np.ascontiguousarray(table_row, dtype=np.int32)
    hq, hkv = q_row.shape[0], k_pool.shape[1]
    out = np.zeros((hq, 128), dtype=np.float32)
    lib().pkv_oracle_paged_decode(q_row, k_pool, v_pool, table_row, hq, hkv, page_size, length,
                                  num_splits, out)
    return out


def split_partial(q_head, k_pool, v_pool, table_row, page_size, kvh, length, tile_begin, tile_end):
    """fp32 partial state ``(m, l, acc[128])`` of one query head over a tile range."""
    m, l = ctypes.c_float(), ctypes.c_float()
    acc = np.zeros(128, dtype=np.float32)
    lib().pkv_oracle_split_partial(np.ascontiguousarray(q_head, dtype=np.float32),
                                   np.ascontiguousarray(k_pool, dtype=np.float32),
                                   np.ascontiguousarray(v_pool, dtype=np.float32),
                                   np.ascontiguousarray(table_row, dtype=np.int32),
                                   k_pool.shape[1], page_size, kvh, length, tile_begin, tile_end,
                                   ctypes.byref(m), ctypes.byref(l), acc)
    return m.value, l.value, acc


def cpu_gqa_attention(q, k, v):
    """tests/smoke_test.cu:35-74 on contiguous fp32 ``q [B,Hq,d]``, ``k/v [B,Hkv,N,d]``."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    b, hq, d = q.shape
    hkv, n = k.shape[1], k.shape[2]
    out = np.zeros((b, hq, d), dtype=np.float32)
    lib().pkv_oracle_cpu_gqa_attention(q, k, v, out, b, hq, hkv, n, d)
    return out


SMOKE_CASES = 8


def smoke_case(index):
    """``(B, Hq, Hkv, N, splits, page_size)`` of smoke case ``index`` (page_size 0 =
    the contiguous layout)."""
    buf = (ctypes.c_int * 6)()
    if lib().pkv_oracle_smoke_case(index, buf) != 0:
        raise IndexError(index)
    return tuple(buf)


def smoke_inputs(index):
    """fp32 Q, K, V of smoke case ``index`` as drawn by glibc ``rand()`` after
    ``srand(42)`` (tests/smoke_test.cu:77-81, :438)."""
    b, hq, hkv, n, _, _ = smoke_case(index)
    q = np.zeros((b, hq, 128), dtype=np.float32)
    k = np.zeros((b, hkv, n, 128), dtype=np.float32)
    v = np.zeros((b, hkv, n, 128), dtype=np.float32)
    lib().pkv_oracle_smoke_inputs(index, q, k, v)
    return q, k, v
