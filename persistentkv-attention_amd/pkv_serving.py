"""Serving-trace engine loop of the PersistentKV engine: the counterpart of the step
runners, router, route profiles, timing and correctness gate of
tests/benchmark_serving_trace.py (ahmed123hds/persistentkv-attention).

  length buckets   compile_bucket_step / run_bucket_step: rows grouped by rounded
                   length, one paged_attention_indexed launch per bucket
                   (compile_persistentkv_metadata :731-780, run_persistentkv_step_compiled
                   :986-1000); metadata from the host C++ builder pkv_build_buckets
  work queue       pkv_workloads.compile_step / run_step (:668-729, :967-984)
  adaptive engine  every step routed by the MI355X cost model (pkv_choose_adaptive_route,
                   policy MI355X) to the split grid or the work queue, as adaptive_step
                   routes it (:1413-1419) -- never to a FlashInfer route, which this
                   engine does not have
  route profiles   launches, non-empty CTA fraction, decode CTAs per CU, useful KV MB and
                   merge-state MB per step (bucket_profile / workqueue_profile /
                   adaptive_profile :516-616)
  timing           per-step HIP-event and synchronised wall time, mean / p50 / p95 / p99
                   and tokens per second (benchmark_engine :1039-1079,
                   summarize_step_latencies :1029-1036)
  gate             one sampled step against a torch fp32 SDPA of the same pages on the
                   GPU, outside the timed region (max-abs 2e-3, mean-abs 3e-4;
                   correctness_check :1082-1088, applied at :1432-1437, where the
                   reference compares against FlashInfer)

Differences from the reference, on purpose:
  * one execution per measured step gives both its event and its wall time (the
    reference runs every step twice, once per clock, :1054-1055);
  * a bucket whose requested split count exceeds its 32-token tiles runs with as many
    splits as it has tiles (the reference op would reject it, cuh:1042-1043);
  * the KV pool can be rotated over replicas between steps (HBM-cold; ``--rotations``),
    where the reference reuses one pool.

Command line (GPU):  python pkv_serving.py --workload c4 [--workload c3_32k ...]
                      [--engines bucket workqueue adaptive] [--repeats 1] [--kv-fp8]
                      [--graph] [--json F] [--md F]
A trace of the reference's harness, with its options and defaults:
                     python pkv_serving.py --trace bimodal --requests 24 --max-active 8
                      --steps 48 --hole-fraction 0.0 --seed 20260623 --workqueue-splits 20
                      [--trace-file F] [--page-size 16] [--hkv 8] [--bucket-tokens 0]
                      [--bucket-splits 32] [--rotations 1] [--graph]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from dataclasses import dataclass

import numpy as np
import torch

import pkv_native
import pkv_workloads as wl

HEAD_DIM = 128
MAX_ABS = 2e-3
MEAN_ABS = 3e-4  # the reference's mean gate (benchmark_serving_trace.py:37-38)
COMPUTE_UNITS = 256


# ---------------------------------------------------------------------------------
# Correctness gate: torch fp32 attention over the same pages, on the GPU.
# ---------------------------------------------------------------------------------
def dequantize_pool(pool, scale):
    """fp8 (float8_e4m3fn) pages as fp32 values scale * e4m3 (torch's exact decode)."""
    return pool.float() * scale


def append_reference(w, meta, k_pages, v_pages, new_kv):
    """Writes each row's new token at position seq_lens - 1 into its tail page, as
    append_kv does (rows with no tokens, a position past the table or a page id outside
    the pool are skipped); fp8 workloads store scale * e4m3(x / scale) into the fp32
    pools given here."""
    k_new, v_new = new_kv
    lens = meta.seq_lens.tolist()
    table = meta.block_table.cpu()
    ps = w.page_size
    for b, n in enumerate(lens):
        pos = n - 1
        if pos < 0 or pos // ps >= table.shape[1]:
            continue
        page = int(table[b, pos // ps])
        if page < 0 or page >= k_pages.shape[0]:
            continue
        kn, vn = k_new[b].float(), v_new[b].float()
        if w.kv_fp8:
            kn = (kn / w.k_scale).clamp(-448, 448).to(torch.float8_e4m3fn).float() * w.k_scale
            vn = (vn / w.v_scale).clamp(-448, 448).to(torch.float8_e4m3fn).float() * w.v_scale
        k_pages[page, :, pos % ps] = kn.to(k_pages.dtype)
        v_pages[page, :, pos % ps] = vn.to(v_pages.dtype)


def reference_step(meta, q_source, k_pages, v_pages, page_size):
    """fp32 decode attention of one step's rows on the device: the row's pages gathered
    through its block table, softmax(q k^T / sqrt(128)) v per KV head group.  Returns
    [output rows, Hq, 128] in the output's row order (out_indices)."""
    lens = meta.seq_lens.tolist()
    q_idx = meta.q_indices.tolist()
    o_idx = meta.out_indices.tolist()
    hq = q_source.shape[1]
    hkv = k_pages.shape[1]
    group = hq // hkv
    cap = meta.block_table.shape[1] * page_size
    out = torch.zeros(meta.output.shape[0], hq, HEAD_DIM, dtype=torch.float32,
                      device=q_source.device)
    scale = 1.0 / math.sqrt(HEAD_DIM)
    for b, n in enumerate(lens):
        n = min(max(n, 0), cap)
        if n == 0:
            continue
        pages = meta.block_table[b, : -(-n // page_size)].long().clamp(0, k_pages.shape[0] - 1)
        k = k_pages.index_select(0, pages).float().permute(1, 0, 2, 3).reshape(hkv, -1, HEAD_DIM)[:, :n]
        v = v_pages.index_select(0, pages).float().permute(1, 0, 2, 3).reshape(hkv, -1, HEAD_DIM)[:, :n]
        q = q_source[q_idx[b]].float().reshape(hkv, group, HEAD_DIM)
        s = torch.matmul(q, k.transpose(1, 2).contiguous()) * scale
        o = torch.matmul(torch.softmax(s, dim=-1), v.contiguous())
        out[o_idx[b]] = o.reshape(hq, HEAD_DIM)
    return out


def gate_step(out, meta, q_source, k_pages, v_pages, page_size):
    """Max-abs / mean-abs of one step's output against reference_step.  bf16 outputs carry
    8 significant bits, so their max-abs bound adds half a bf16 ulp of |ref| (the raw
    max-abs is reported too) and their mean is taken against the bf16-rounded reference."""
    ref = reference_step(meta, q_source, k_pages, v_pages, page_size)
    got = out.float()
    diff = (got - ref).abs()
    res = {"max_abs": float(diff.max()), "mean_abs": float(diff.mean()),
           "bound": f"max-abs < {MAX_ABS}, mean-abs < {MEAN_ABS} vs torch fp32 on the GPU"}
    ok = torch.isfinite(got).all().item()
    if out.dtype == torch.bfloat16:
        mag = ref.abs().clamp_min(2.0 ** -126)
        half_ulp = torch.exp2(torch.floor(torch.log2(mag)) - 8)
        res["max_abs_over_half_bf16_ulp"] = float((diff - half_ulp).max())
        res["mean_abs_vs_bf16_rounded"] = float((got - ref.to(torch.bfloat16).float()).abs().mean())
        ok = ok and res["max_abs_over_half_bf16_ulp"] < MAX_ABS and res["mean_abs_vs_bf16_rounded"] < MEAN_ABS
    else:
        ok = ok and res["max_abs"] < MAX_ABS and res["mean_abs"] < MEAN_ABS
    res["pass"] = bool(ok)
    return res


# ---------------------------------------------------------------------------------
# Length-bucket route.
# ---------------------------------------------------------------------------------
@dataclass
class Bucket:
    bucket_length: int
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    q_indices: torch.Tensor
    out_indices: torch.Tensor
    splits: int            # as the builder chose them (choose_splits)
    launch_splits: int     # at most the bucket's 32-token tiles


@dataclass
class BucketStep:
    buckets: list
    output: torch.Tensor
    kv_bytes: int


def compile_bucket_step(w, step_index, device, requested_splits, auto_splits=False,
                        bucket_tokens=0, single_bucket=False, adaptive_route=False,
                        policy=pkv_native.POLICY_REFERENCE):
    """One step's buckets from the host C++ builder (pkv_build_buckets), on ``device``."""
    st = w.steps[step_index]
    by_id = {r.request_id: r for r in w.requests}
    page_lists = [by_id[i].physical_pages for i in st.active_ids]
    raw = pkv_native.build_buckets(list(st.lengths), list(st.active_ids), page_lists, w.page_size,
                                   requested_splits, auto_splits, bucket_tokens, single_bucket,
                                   adaptive_route, w.hkv, policy)
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32).to(device)
    buckets = []
    for b in raw:
        tiles = max(1, -(-b["bucket_length"] // 32))
        buckets.append(Bucket(b["bucket_length"], t(b["block_table"]), t(b["seq_lens"]),
                              t(b["q_indices"]), t(b["out_indices"]), b["splits"],
                              max(1, min(b["splits"], tiles))))
    output = torch.empty(len(st.active_ids), w.hq, HEAD_DIM, device=device, dtype=w.dtype)
    return BucketStep(buckets, output, w.kv_bytes(step_index))


def bucket_workspace(w, steps, device):
    """fp32 workspace for every bucket launch of ``steps`` (split partial states with room
    for a few-unit launch's sub-splits, or the direct launch's internal split)."""
    floats = 1
    for s in steps:
        for b in s.buckets:
            rows = int(b.seq_lens.numel())
            if b.launch_splits > 1:
                floats = max(floats, pkv_native.split_workspace_bytes(
                    rows, w.hq, w.hkv, b.bucket_length, b.launch_splits) // 4)
            else:
                floats = max(floats, pkv_native.direct_workspace_bytes(rows, w.hq, w.hkv,
                                                                       b.bucket_length) // 4)
    return torch.empty(floats, device=device, dtype=torch.float32)


def run_bucket_step(ext, w, step, step_index, q_pool, k_pages, v_pages, workspace):
    """One paged_attention_indexed launch per bucket into the step's output
    (run_persistentkv_step_compiled, benchmark_serving_trace.py:986-1000)."""
    q_source = q_pool[step_index]
    for b in step.buckets:
        if w.kv_fp8:
            ext.paged_attention_indexed_fp8(q_source, k_pages, v_pages, b.block_table, b.seq_lens,
                                            b.q_indices, b.out_indices, step.output, workspace,
                                            b.bucket_length, w.page_size, b.launch_splits,
                                            w.k_scale, w.v_scale)
        else:
            ext.paged_attention_indexed(q_source, k_pages, v_pages, b.block_table, b.seq_lens,
                                        b.q_indices, b.out_indices, step.output, workspace,
                                        b.bucket_length, w.page_size, b.launch_splits)
    return step.output


# ---------------------------------------------------------------------------------
# Engines: fixed length buckets, fixed work queue, adaptive.
# ---------------------------------------------------------------------------------
def mi355x_model(w):
    return pkv_native.cost_model(pkv_native.POLICY_MI355X, num_q_heads=w.hq, num_kv_heads=w.hkv)


class Engine:
    """Per-step metadata of one engine over a workload, compiled before timing (as the
    reference's --precompute-metadata does, :1288-1327).

    ``bucket``     exact-length buckets with the workload's split rule (the reference's
                   length-bucket engine)
    ``workqueue``  the compact work queue with the workload's split rule
    ``adaptive``   each step routed by the MI355X cost model: the split grid as one
                   ragged bucket with the router's split count, or the work queue with
                   the MI355X split planner
    """

    def __init__(self, name, w, device, splits=None, bucket_tokens=0):
        self.name, self.w, self.device = name, w, device
        n = len(w.steps)
        self.routes = []
        self.meta = []
        fixed = w.splits if splits is None else splits
        for i in range(n):
            if name == "bucket":
                route, splits = "persistentkv_bucket", fixed
            elif name == "workqueue":
                route, splits = "persistentkv_workqueue", fixed
            elif name == "adaptive":
                route, splits, _ = pkv_native.choose_adaptive_route(list(w.steps[i].lengths),
                                                                    mi355x_model(w))
            else:
                raise ValueError(f"unknown engine {name}")
            self.routes.append((route, splits))
            if route == "persistentkv_workqueue":
                saved = (w.splits, w.auto_splits, w.policy)
                if name == "adaptive":
                    w.splits, w.auto_splits, w.policy = 1, True, pkv_native.POLICY_MI355X
                else:
                    w.splits = fixed
                m = _queue_step(w, i, device)
                w.splits, w.auto_splits, w.policy = saved
                self.meta.append(("queue", m))
            else:
                if name == "adaptive":
                    step = compile_bucket_step(w, i, device, splits, single_bucket=True,
                                               bucket_tokens=bucket_tokens)
                else:
                    step = compile_bucket_step(w, i, device, fixed, auto_splits=w.auto_splits,
                                               bucket_tokens=bucket_tokens, policy=w.policy)
                self.meta.append(("bucket", step))
        queue_metas = [m for kind, m in self.meta if kind == "queue"]
        bucket_steps = [m for kind, m in self.meta if kind == "bucket"]
        floats = 1
        if queue_metas:
            floats = max(floats, wl.workspace_for(w, queue_metas, "meta").numel())
        if bucket_steps:
            floats = max(floats, bucket_workspace(w, bucket_steps, "meta").numel())
        self.workspace = torch.empty(floats, device=device, dtype=torch.float32)

    def output(self, i):
        kind, m = self.meta[i]
        return m.output

    def run(self, ext, i, q_pool, k_pages, v_pages):
        kind, m = self.meta[i]
        if kind == "queue":
            return wl.run_step(ext, self.w, m, i, q_pool, k_pages, v_pages, self.workspace)
        return run_bucket_step(ext, self.w, m, i, q_pool, k_pages, v_pages, self.workspace)

    def gate_meta(self, i):
        """A StepMeta-like view (block table, lengths, indices, output) of step i's rows
        for the gate: the work-queue step's own metadata, or the buckets stacked."""
        kind, m = self.meta[i]
        if kind == "queue":
            return m
        cols = max(int(b.block_table.shape[1]) for b in m.buckets)
        tables, lens, qi, oi = [], [], [], []
        for b in m.buckets:
            t = b.block_table
            if t.shape[1] < cols:
                t = torch.cat([t, t[:, -1:].expand(-1, cols - t.shape[1])], dim=1)
            tables.append(t)
            lens.append(b.seq_lens)
            qi.append(b.q_indices)
            oi.append(b.out_indices)
        return _GateMeta(torch.cat(tables), torch.cat(lens), torch.cat(qi), torch.cat(oi), m.output)


@dataclass
class _GateMeta:
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    q_indices: torch.Tensor
    out_indices: torch.Tensor
    output: torch.Tensor


def _queue_step(w, i, device):
    """Work-queue metadata of step i (pkv_workloads.compile_step with the op forced to the
    work queue)."""
    op = w.op
    w.op = "paged_attention_workqueue"
    try:
        return wl.compile_step(w, i, device)
    finally:
        w.op = op


# ---------------------------------------------------------------------------------
# Structural route profiles (benchmark_serving_trace.py:516-616).
# ---------------------------------------------------------------------------------
def _mb(nbytes):
    return nbytes / (1024.0 * 1024.0)


def step_profile(w, kind, m, fused_merge=False):
    """(launches, nonempty CTA fraction, decode CTAs per CU, merge-state MB, merge launches)
    of one compiled step."""
    if kind == "queue":
        items = int(m.num_tasks)
        return (1 if fused_merge else 2, 1.0, items / COMPUTE_UNITS,
                _mb(m.total_partial_slots * w.hq * (2 + HEAD_DIM) * 4), 0 if fused_merge else 1)
    launches = possible = nonempty = ctas = merge_bytes = merge_launches = 0
    for b in m.buckets:
        rows = int(b.seq_lens.numel())
        s = b.launch_splits
        launches += 1 if s == 1 else 2
        ctas += rows * w.hkv * s
        possible += rows * w.hkv * s
        for n in b.seq_lens.tolist():
            tiles = (n + 31) // 32
            nonempty += w.hkv * sum(1 for k in range(s) if (tiles * k) // s < (tiles * (k + 1)) // s)
        if s > 1:
            merge_launches += 1
            merge_bytes += rows * w.hq * s * (2 + HEAD_DIM) * 4
    return (launches, nonempty / max(1, possible), ctas / COMPUTE_UNITS, _mb(merge_bytes),
            merge_launches)


def engine_profile(engine, fused_merge=False):
    w = engine.w
    rows = [step_profile(w, kind, m, fused_merge) for kind, m in engine.meta]
    keys = ("launches_per_step", "nonempty_cta_fraction", "decode_ctas_per_cu",
            "merge_state_mb", "merge_launches_per_step")
    prof = {k: statistics.mean(r[j] for r in rows) for j, k in enumerate(keys)}
    prof["useful_kv_read_mb"] = statistics.mean(_mb(w.kv_bytes(i)) for i in range(len(w.steps)))
    routes = [r for r, _ in engine.routes]
    prof["route_counts"] = {r: routes.count(r) for r in sorted(set(routes))}
    prof["route_splits"] = {r: sorted({s for rr, s in engine.routes if rr == r}) for r in set(routes)}
    return prof


# ---------------------------------------------------------------------------------
# Timing (benchmark_serving_trace.py:1004-1079).
# ---------------------------------------------------------------------------------
def summarize(samples):
    """(mean, p50, p95, p99) with the reference's percentile rule: the ceil(p * n)-th
    smallest sample (summarize_step_latencies, :1029-1036)."""
    ordered = sorted(samples)
    if not ordered:
        return 0.0, 0.0, 0.0, 0.0

    def pct(p):
        return ordered[min(len(ordered) - 1, int(math.ceil(p * len(ordered)) - 1))]
    return statistics.mean(ordered), pct(0.50), pct(0.95), pct(0.99)


def benchmark_engine(step_fn, w, warmup_steps, repeats):
    """Per-step event and wall timing over ``repeats`` passes of the trace.  ``step_fn(k,
    i)`` runs timed call k on trace step i.  Each step is synchronised before and after,
    and one execution gives both clocks."""
    n = len(w.steps)
    for k in range(min(warmup_steps, n)):
        step_fn(k, k)
    torch.cuda.synchronize()
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    event_ms, wall_ms = [], []
    k = 0
    for _ in range(repeats):
        for i in range(n):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            ev0.record()
            step_fn(k, i)
            ev1.record()
            ev1.synchronize()
            wall_ms.append((time.perf_counter() - t0) * 1e3)
            event_ms.append(ev0.elapsed_time(ev1))
            k += 1
    tokens = sum(len(s.active_ids) for s in w.steps) * repeats
    e = summarize(event_ms)
    wa = summarize(wall_ms)
    kv = sum(w.kv_bytes(i) for i in range(n)) * repeats
    return {"tokens": tokens, "steps": len(event_ms),
            "event_tokens_s": tokens / (sum(event_ms) / 1e3),
            "wall_tokens_s": tokens / (sum(wall_ms) / 1e3),
            "event_mean_ms": e[0], "event_p50_ms": e[1], "event_p95_ms": e[2], "event_p99_ms": e[3],
            "wall_mean_ms": wa[0], "wall_p50_ms": wa[1], "wall_p95_ms": wa[2], "wall_p99_ms": wa[3],
            "event_kv_gbps": kv / (sum(event_ms) / 1e3) / 1e9}


# ---------------------------------------------------------------------------------
# Driver.
# ---------------------------------------------------------------------------------
def run_workload(ext, name, engines, repeats, warmup, rotations, device, seed, kv_fp8=False,
                 w=None, engine_splits=None, bucket_tokens=0, graph=False):
    """Gates and times ``engines`` over a workload: a named configuration, or ``w`` (a
    trace of the reference's harness, with ``engine_splits`` = {engine: split count} and
    ``bucket_tokens`` as its --adaptive-*-splits and --bucket-tokens).  With ``graph``
    each step is captured once into a HIP graph and replayed (the reference's
    --pkv-cuda-graph, :1439-1452)."""
    if w is None:
        w = wl.CONFIGS[name](seed=seed)
    w.kv_fp8 = kv_fp8
    engine_splits = engine_splits or {}
    q_pool = wl.make_q_pool(w, device)
    k0, v0 = wl.make_kv_pool(w, device)
    pools = [(k0, v0)] + [(k0.clone(), v0.clone()) for _ in range(max(1, rotations) - 1)]
    report = {"workload": name, "hq": w.hq, "hkv": w.hkv, "page_size": w.page_size,
              "dtype": str(w.dtype).replace("torch.", "") + (" (fp8 e4m3 K/V)" if kv_fp8 else ""),
              "trace_steps": len(w.steps),
              "requests": len(w.requests), "repeats": repeats,
              "active_mean": statistics.mean(len(s.active_ids) for s in w.steps),
              "useful_kv_mb_per_step": statistics.mean(_mb(w.kv_bytes(i)) for i in range(len(w.steps))),
              "cache_basis": f"{len(pools)} KV pool replica(s) rotated per step",
              "launch": "hip graph per step" if graph else "eager", "engines": {}}
    if w.extra.get("trace") is not None:
        report["trace"] = {k: w.extra[k] for k in ("trace", "max_active", "hole_fraction",
                                                   "bucket_tokens", "trace_file")}
        report["trace"]["seed"] = w.seed
        report["physical_pages"] = w.physical_pages
    for name_e in engines:
        eng = Engine(name_e, w, device, splits=engine_splits.get(name_e),
                     bucket_tokens=bucket_tokens)
        gi = len(w.steps) // 2
        out = eng.run(ext, gi, q_pool, k0, v0).clone()
        torch.cuda.synchronize()
        kd, vd = ((dequantize_pool(k0, w.k_scale), dequantize_pool(v0, w.v_scale)) if w.kv_fp8
                  else (k0, v0))
        gate = gate_step(out, eng.gate_meta(gi), q_pool[gi], kd, vd, w.page_size)
        gate["step"] = gi
        del kd, vd
        if not gate["pass"]:
            raise SystemExit(f"{name}/{name_e}: correctness gate failed at step {gi}: {gate}")

        if graph:
            # One graph per trace step, each over the pool replica the step's first timed
            # call would use (warm-up runs first, outside capture).
            graphs = []
            for i in range(len(w.steps)):
                kp, vp = pools[i % len(pools)]
                eng.run(ext, i, q_pool, kp, vp)
                torch.cuda.synchronize()
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g):
                    eng.run(ext, i, q_pool, kp, vp)
                graphs.append(g)
            torch.cuda.synchronize()

            def step_fn(k, i):
                graphs[i].replay()
        else:
            def step_fn(k, i):
                kp, vp = pools[k % len(pools)]
                eng.run(ext, i, q_pool, kp, vp)
        stats = benchmark_engine(step_fn, w, warmup, repeats)
        report["engines"][name_e] = {"stats": stats, "profile": engine_profile(eng, w.fused_merge),
                                     "gate": gate}
        if graph:
            del graphs
        print(f"{name:8s} {name_e:10s} event mean {stats['event_mean_ms'] * 1e3:8.1f} us "
              f"p95 {stats['event_p95_ms'] * 1e3:8.1f} us  {stats['event_tokens_s']:10.0f} tok/s  "
              f"gate max {gate['max_abs']:.2e}", flush=True)
        del eng
    return report


def calibrate(ext, device, steps_per_workload=6, reps=5, rotations=4):
    """Step times of the two routes the MI355X router chooses between, on sampled steps of
    this engine's configurations and the reference's review traces: the split grid as one
    ragged bucket with the router's split count (pkv_model_bucket_splits) and the work
    queue with the MI355X planner.  Each time is the mean of ``reps`` event-timed calls,
    HBM-cold (pool replicas rotated), after two warm-up calls.  pkv_calibrate.py fits the
    cost model's constants to these samples."""
    cases = [(name, lambda name=name: wl.CONFIGS[name]())
             for name in ("c1", "c2", "c3", "c3_32k", "c4", "c5_g8", "c5_g32")]
    for trace, b, reqs, steps, hkv in (("bimodal", 8, 24, 48, 8), ("bimodal", 8, 24, 48, 4),
                                       ("bimodal", 8, 24, 48, 32), ("uniform", 8, 24, 48, 8),
                                       ("zipf", 8, 24, 48, 8), ("bucketed", 1, 16, 64, 8),
                                       ("homogeneous", 4, 8, 48, 8)):
        cases.append((f"trace_{trace}_b{b}_hkv{hkv}",
                      lambda t=trace, b=b, r=reqs, n=steps, h=hkv:
                      wl.config_trace(t, r, b, n, 20260623, 0.0, 16, h, 32, 16)))
    samples = []
    for name, make in cases:
        w = make()
        q_pool = wl.make_q_pool(w, device)
        k0, v0 = wl.make_kv_pool(w, device)
        pools = [(k0, v0)] + [(k0.clone(), v0.clone()) for _ in range(rotations - 1)]
        n = len(w.steps)
        picks = sorted({(j * n) // steps_per_workload for j in range(steps_per_workload)})
        model = mi355x_model(w)
        for i in picks:
            lengths = list(w.steps[i].lengths)
            bs = pkv_native.model_bucket_splits(lengths, w.hkv, pkv_native.POLICY_MI355X)
            grid = compile_bucket_step(w, i, device, bs, single_bucket=True)
            gws = bucket_workspace(w, [grid], device)
            saved = (w.splits, w.auto_splits, w.policy)
            w.splits, w.auto_splits, w.policy = 1, True, pkv_native.POLICY_MI355X
            queue = _queue_step(w, i, device)
            w.splits, w.auto_splits, w.policy = saved
            qws = wl.workspace_for(w, [queue], device)

            def timed(fn):
                for k in range(2):
                    fn(*pools[k % len(pools)])
                torch.cuda.synchronize()
                ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                      for _ in range(reps)]
                for k in range(reps):
                    kp, vp = pools[(k + 2) % len(pools)]
                    ev[k][0].record()
                    fn(kp, vp)
                    ev[k][1].record()
                torch.cuda.synchronize()
                return statistics.mean(a.elapsed_time(b) * 1e3 for a, b in ev)

            grid_us = timed(lambda kp, vp: run_bucket_step(ext, w, grid, i, q_pool, kp, vp, gws))
            queue_us = timed(lambda kp, vp: wl.run_step(ext, w, queue, i, q_pool, kp, vp, qws))
            route, _, _ = pkv_native.choose_adaptive_route(lengths, model)
            samples.append({"workload": name, "step": i, "hq": w.hq, "hkv": w.hkv,
                            "dtype": str(w.dtype).replace("torch.", ""), "lengths": lengths,
                            "grid_splits": bs, "grid_us": round(grid_us, 2),
                            "queue_us": round(queue_us, 2), "router_at_run": route})
            print(f"{name:24s} step {i:3d} grid S={bs:3d} {grid_us:8.1f} us  queue {queue_us:8.1f} us"
                  f"  router {route}", flush=True)
        del pools, k0, v0, q_pool
        torch.cuda.empty_cache()
    return samples


def markdown(reports):
    lines = []
    for r in reports:
        tr = r.get("trace")
        head = r["workload"]
        if tr:
            head = (f"trace={tr['trace'] if not tr['trace_file'] else tr['trace_file']} "
                    f"seed={tr['seed']} requests={r['requests']} max_active={tr['max_active']} "
                    f"hole_fraction={tr['hole_fraction']:.2f} bucket_tokens={tr['bucket_tokens']} "
                    f"physical_pages={r['physical_pages']}")
        lines += [f"### {head}  (Hq {r['hq']} / Hkv {r['hkv']}, page {r['page_size']}, "
                  f"{r['dtype']}, {r['trace_steps']} steps x {r['repeats']}, mean active "
                  f"{r['active_mean']:.2f}, {r['useful_kv_mb_per_step']:.1f} MiB useful KV per "
                  f"step, {r['cache_basis']}, {r['launch']})", "",
                  "| Engine | GPU tokens/s | GPU mean step us | GPU p50 us | GPU p95 us | GPU p99 us "
                  "| Wall tokens/s | Wall mean us | Wall p95 us | KV GB/s (event) | gate max-abs |",
                  "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
        for name, e in r["engines"].items():
            s, g = e["stats"], e["gate"]
            lines.append(f"| {name} | {s['event_tokens_s']:.0f} | {s['event_mean_ms'] * 1e3:.1f} | "
                         f"{s['event_p50_ms'] * 1e3:.1f} | {s['event_p95_ms'] * 1e3:.1f} | "
                         f"{s['event_p99_ms'] * 1e3:.1f} | {s['wall_tokens_s']:.0f} | "
                         f"{s['wall_mean_ms'] * 1e3:.1f} | {s['wall_p95_ms'] * 1e3:.1f} | "
                         f"{s['event_kv_gbps']:.0f} | {g['max_abs']:.2e} |")
        lines += ["", "| Engine | launches/step | non-empty CTA fraction | decode CTAs per CU | "
                  "useful KV MiB/step | merge-state MiB/step | merge launches/step | routes |",
                  "|---|---:|---:|---:|---:|---:|---:|---|"]
        for name, e in r["engines"].items():
            p = e["profile"]
            routes = ", ".join(f"{k}={v} (splits {p['route_splits'][k]})"
                               for k, v in p["route_counts"].items())
            lines.append(f"| {name} | {p['launches_per_step']:.2f} | {p['nonempty_cta_fraction']:.3f} | "
                         f"{p['decode_ctas_per_cu']:.2f} | {p['useful_kv_read_mb']:.1f} | "
                         f"{p['merge_state_mb']:.2f} | {p['merge_launches_per_step']:.2f} | {routes} |")
        lines.append("")
    return "\n".join(lines)


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--workload", action="append", choices=sorted(wl.CONFIGS),
                   help="configuration(s) to run (default: c1 c2 c3 c3_32k c4 c5_g8 c5_g32)")
    # A trace of the reference's harness, with its options and defaults
    # (benchmark_serving_trace.py:1114-1211); replaces --workload when given.
    p.add_argument("--trace", choices=["uniform", "bimodal", "zipf", "bucketed", "homogeneous"])
    p.add_argument("--trace-file", help="CSV/JSON request trace (prompt_len/prompt, "
                                        "decode_len/decode, optional arrival/arrival_step)")
    p.add_argument("--requests", type=int, default=24)
    p.add_argument("--max-active", type=int, default=8)
    p.add_argument("--steps", type=int, default=48)
    p.add_argument("--hole-fraction", type=float, default=0.50)
    p.add_argument("--page-size", type=int, choices=[16, 32, 64, 128], default=16)
    p.add_argument("--hkv", type=int, default=8, choices=[1, 2, 4, 8, 16, 32],
                   help="KV heads; Hq is 32, so G = 32 / hkv")
    p.add_argument("--bucket-tokens", type=int, default=0,
                   help="round the length-bucket route's lengths up to this many tokens")
    p.add_argument("--bucket-splits", type=int, default=32,
                   help="split count of the length-bucket engine (the reference's "
                        "--adaptive-bucket-splits)")
    p.add_argument("--workqueue-splits", type=int, default=24,
                   help="split count of the work-queue engine (the reference's "
                        "--adaptive-workqueue-splits)")
    p.add_argument("--graph", action="store_true",
                   help="capture each step in a HIP graph and replay it (--pkv-cuda-graph)")
    p.add_argument("--engines", nargs="+", default=["bucket", "workqueue", "adaptive"],
                   choices=["bucket", "workqueue", "adaptive"])
    p.add_argument("--repeats", type=int, default=1)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--rotations", type=int, default=4,
                   help="KV pool replicas rotated per step (1 reuses one pool, as the reference)")
    p.add_argument("--seed", type=int, default=None,
                   help="default: the configurations' seed, or 20260622 for a trace (the "
                        "reference harness's default)")
    p.add_argument("--kv-fp8", action="store_true",
                   help="K/V pools in fp8 (OCP e4m3) with the workload's per-tensor scales; every "
                        "engine runs the *_fp8 ops and the gate uses the dequantised pages")
    p.add_argument("--json")
    p.add_argument("--md")
    p.add_argument("--calibrate", metavar="FILE",
                   help="time the router's two routes on sampled steps of every configuration "
                        "and review trace and write the samples to FILE (pkv_calibrate.py fits "
                        "the MI355X cost model to them)")
    a = p.parse_args(argv)
    import persistentkv_torch_ext as ext
    device = torch.device("cuda:0")
    if a.calibrate:
        samples = calibrate(ext, device)
        with open(a.calibrate, "w") as fh:
            json.dump({"gpu": torch.cuda.get_device_name(0), "compute_units": COMPUTE_UNITS,
                       "samples": samples}, fh, indent=1)
        return
    reports = []
    if a.trace or a.trace_file:
        seed = 20260622 if a.seed is None else a.seed
        w = wl.config_trace(a.trace or "bimodal", a.requests, a.max_active, a.steps, seed,
                            a.hole_fraction, a.page_size, a.hkv, 32, a.workqueue_splits,
                            a.bucket_tokens, a.trace_file)
        splits = {"bucket": a.bucket_splits, "workqueue": a.workqueue_splits}
        reports.append(run_workload(ext, w.name, a.engines, a.repeats, a.warmup, a.rotations,
                                    device, seed, a.kv_fp8, w=w, engine_splits=splits,
                                    bucket_tokens=a.bucket_tokens, graph=a.graph))
    else:
        names = a.workload or ["c1", "c2", "c3", "c3_32k", "c4", "c5_g8", "c5_g32"]
        for name in names:
            reports.append(run_workload(ext, name, a.engines, a.repeats, a.warmup, a.rotations,
                                        device, wl.DEFAULT_SEED if a.seed is None else a.seed,
                                        a.kv_fp8, graph=a.graph))
            torch.cuda.empty_cache()
    text = markdown(reports)
    print(text, flush=True)
    if a.json:
        with open(a.json, "w") as fh:
            json.dump({"gpu": torch.cuda.get_device_name(0), "reports": reports}, fh, indent=1)
    if a.md:
        with open(a.md, "w") as fh:
            fh.write(text + "\n")


if __name__ == "__main__":
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    main()
