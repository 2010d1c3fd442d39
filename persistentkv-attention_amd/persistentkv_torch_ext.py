"""PersistentKV paged decode attention for MI355X — PyTorch op surface.

Drop-in for the module that tests/benchmark_serving_trace.py builds with
``torch.utils.cpp_extension.load(name="persistentkv_torch_ext", ...)`` (:133-156): the
same four ops with the same positional arguments, checks and in-place ``None`` return
(tests/persistentkv_torch_extension.cu:319-336), backed by the HIP engine in
``libpkv.so``.  Import it after adding this directory to ``sys.path``.

``import torch`` comes first so that the native library binds to the HIP runtime torch
already loaded.  There is no CPU fallback: importing fails if the native extension has
not been built.
"""
from __future__ import annotations

import importlib.util
import os
import sysconfig

import torch  # noqa: F401  (must precede the native library, see the docstring)

_HERE = os.path.dirname(os.path.abspath(__file__))
EXTENSION_PATH = os.path.join(_HERE, "_pkv_torch" + sysconfig.get_config_var("EXT_SUFFIX"))
LIBRARY_PATH = os.path.join(_HERE, "libpkv.so")


def _load():
    for path in (LIBRARY_PATH, EXTENSION_PATH):
        if not os.path.exists(path):
            raise ImportError(
                f"PersistentKV native code is not built ({path} missing); run "
                "`python -c 'import __graft_entry__ as g; g.build()'` or "
                "`make -C persistentkv-attention_amd/csrc`")
    spec = importlib.util.spec_from_file_location("_pkv_torch", EXTENSION_PATH)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


_ext = _load()

paged_attention = _ext.paged_attention
paged_attention_masked = _ext.paged_attention_masked
paged_attention_indexed = _ext.paged_attention_indexed
paged_attention_workqueue = _ext.paged_attention_workqueue
workqueue_decode = _ext.workqueue_decode
workqueue_merge = _ext.workqueue_merge
# The schedule of paged_attention_workqueue (1 = balanced: equal tile shares per wave over
# every (row, kv head) pair of a complete queue; 0 = one workgroup per work item) for
# (batch, Hq, Hkv, page_size, workspace floats, fused_merge), and one stage of it
# (stage, then the paged_attention_workqueue tensors without merge_counters, then
# bucket_context, page_size, total_partial_slots, kv_fp8, k_scale, v_scale).
workqueue_schedule = _ext.workqueue_schedule
paged_attention_workqueue_stage = _ext.paged_attention_workqueue_stage
# fp8 (float8_e4m3fn) K/V pages with per-tensor scales: K = k_scale * k8, V = v_scale * v8.
paged_attention_indexed_fp8 = _ext.paged_attention_indexed_fp8
paged_attention_workqueue_fp8 = _ext.paged_attention_workqueue_fp8
workqueue_decode_fp8 = _ext.workqueue_decode_fp8
# Contiguous K/V [B, Hkv, N, 128] (the reference's C++ entry points, cuh:1077-1108, 1263-1282).
attention_contiguous = _ext.attention_contiguous
attention_query_head_baseline = _ext.attention_query_head_baseline
# KV-cache append: k_new / v_new [B, Hkv, 128] to position seq_lens[b] - 1 of each row
# (fp8 pools store e4m3(x / scale), rounded to nearest even).
append_kv = _ext.append_kv
append_kv_fp8 = _ext.append_kv_fp8
# The masked, indexed and work-queue ops with that append fused in (2-byte pools): the op's
# arguments followed by k_new, v_new; same result as append_kv then the op.
paged_attention_masked_append = _ext.paged_attention_masked_append
paged_attention_indexed_append = _ext.paged_attention_indexed_append
paged_attention_workqueue_append = _ext.paged_attention_workqueue_append
# The fp8-K/V ops with the append fused in: (..., k_scale, v_scale, k_new, v_new); the new
# token is stored as append_kv_fp8 stores it.
paged_attention_indexed_fp8_append = _ext.paged_attention_indexed_fp8_append
paged_attention_workqueue_fp8_append = _ext.paged_attention_workqueue_fp8_append

# fp32 workspace elements with which a direct (num_splits == 1) launch of paged_attention,
# paged_attention_masked / _indexed or attention_contiguous runs its full internal split
# (0 when it is not split; a smaller workspace gives a smaller split, an empty one none).
direct_workspace_floats = _ext.direct_workspace_floats
split_workspace_floats = _ext.split_workspace_floats

HEAD_DIM = 128
TILE_TOKENS = 32


def workspace_floats(batch: int, num_q_heads: int, num_splits: int) -> int:
    """fp32 workspace elements for a split launch (cuh:891-898; 0 when unsplit)."""
    return 0 if num_splits <= 1 else batch * num_q_heads * num_splits * (2 + HEAD_DIM)


def workqueue_workspace_floats(total_partial_slots: int, num_q_heads: int) -> int:
    """fp32 workspace elements for a work-queue launch (cuh:915-927)."""
    return total_partial_slots * num_q_heads * (2 + HEAD_DIM)


__all__ = [
    "paged_attention", "paged_attention_masked", "paged_attention_indexed",
    "paged_attention_workqueue", "workqueue_decode", "workqueue_merge", "workqueue_schedule",
    "paged_attention_workqueue_stage",
    "paged_attention_indexed_fp8", "paged_attention_workqueue_fp8", "workqueue_decode_fp8",
    "attention_contiguous",
    "attention_query_head_baseline", "append_kv", "append_kv_fp8",
    "paged_attention_masked_append", "paged_attention_indexed_append",
    "paged_attention_workqueue_append",
    "paged_attention_indexed_fp8_append", "paged_attention_workqueue_fp8_append", "workspace_floats",
    "workqueue_workspace_floats", "direct_workspace_floats", "split_workspace_floats", "EXTENSION_PATH", "LIBRARY_PATH",
]
