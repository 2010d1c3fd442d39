"""Benchmark of the MI355X PersistentKV decode engine on its headline workload.

Workload: bimodal continuous-batching trace, 24 requests,
max-active 8, 48 decode steps, Hq 32 / Hkv 8 (G=4), D 128, fp16, page 16, 20 fixed
work-queue splits with metadata precomputed by the host builder.  One "step" is one
``paged_attention_workqueue`` call (decode kernel + LSE merge) over one decode step of
the trace.  The K timed steps are one sample of the trace: whole passes when K is a
multiple of its 48 steps (the default K = 96 is two), otherwise K evenly spaced trace
steps (timed step k replays trace step k * 48 // K).  Every figure of the line (value,
roofline, traffic, mean_kv_mb_per_step) is taken over that same sample.

Cache basis: the KV pool is replicated ``--rotations`` times and consecutive timed steps
read different replicas, so a step's pages have been evicted from the 256 MB Infinity
Cache by the time they are read again (every figure is HBM-cold).

Reported (one JSON line):
  value        effective KV read bandwidth over the timed steps, GB/s (algorithmic
               bytes: sum of active lengths * Hkv * 128 * 2 (K,V) * 2 bytes per step,
               the reference's useful_kv_mb_for_state, tests/benchmark_serving_trace.py:511-513)
  ms_per_step  mean wall time per step between the synchronised bracket points
  roofline     decode kernel alone over the same sample, timed with HIP events on its
               launch stream; traffic = the rocprofv3 FETCH_SIZE + WRITE_SIZE ratio to
               algorithmic bytes (profiles/c4_decode_traffic.json) x the sample's bytes
  gate         one sampled step of the timed op checked against a torch fp32 SDPA of the
               same inputs on the GPU, outside the timed region (max-abs 2e-3, mean-abs
               3e-4; the run fails otherwise)
  cpu_baseline repack + fp32 SDPA (the reference's CPU path, restated in oracle/) on a
               bounded sample of the same steps on the host cores
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "persistentkv-attention_amd")
for _p in (PKG, ROOT):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode-step µs + effective KV HBM GB/s (% of peak), B8 bimodal G=4 fp16"
WORKLOAD_NAMES = {"c1": "c1_b1_ctx2048_direct", "c2": "c2_b8_mha_split8",
                  "c3": "c3_b1_long_context_split32", "c3_32k": "c3_b1_32k_context_split32",
                  "c4": "c4_bimodal_workqueue",
                  "c5_g32": "c5_b64_zipf_mqa_bf16", "c5_g8": "c5_b64_zipf_g8_bf16",
                  "smoke_g4_8k": "smoke_b1_g4_n8192_contiguous_split16",
                  "smoke_g4_32k": "smoke_b1_g4_n32768_contiguous_split16"}
# Published figures of the reference for the same metric and configuration (RTX 3060,
# 360 GB/s peak): results/smoke_test.txt:25 and :27, and every row of its sweep (:23-43).
PUBLISHED_GBPS = {"smoke_g4_8k": 237.1, "smoke_g4_32k": 238.6}
SWEEP = {}  # sweep workload name -> published GB/s (filled from pkv_workloads.SMOKE_SWEEP)


def _sweep_table():
    import pkv_workloads as wl
    for b, hq, hkv, n, splits, gbps in wl.SMOKE_SWEEP:
        for paged in (False, True):
            SWEEP[wl.sweep_name(b, hq, hkv, n, splits, paged)] = gbps


_sweep_table()
HBM_PEAK_GBPS = 8000.0
MALL_BYTES = 256 * 2 ** 20  # MI355X Infinity Cache
WORKSPACE_LABELS = {
    "engine": ("this engine's size for its faster decomposition "
               "(pkv_workqueue_balanced_workspace_bytes / pkv_split_workspace_bytes / "
               "pkv_direct_workspace_bytes, at least the reference's)"),
    "reference": ("the reference callers' size (pkv_workspace_bytes: none for a direct "
                  "launch; total_partial_slots x Hq x 130 floats for the work queue)"),
}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "c4_decode_traffic.json")
TRAFFIC_FILE_FP8 = os.path.join(ROOT, "profiles", "c4_fp8_decode_traffic.json")


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=96)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--rotations", type=int, default=4,
                   help="minimum KV pool replicas (cold-cache basis; raised for small steps)")
    p.add_argument("--workload", default="c4", choices=sorted(WORKLOAD_NAMES) + sorted(SWEEP),
                   help="configuration (default c4, the headline; the others are reported "
                        "for the design notes and are not the metric)")
    p.add_argument("--sweep", action="store_true",
                   help="run the reference's performance sweep (tests/smoke_test.cu:502-521) "
                        "over contiguous and paged K/V, one JSON line per row, each beside "
                        "the reference's published GB/s (no CPU baseline)")
    p.add_argument("--fused-merge", action="store_true", help="single-launch fused merge variant")
    p.add_argument("--kv-fp8", action="store_true",
                   help="K/V pages in fp8 (OCP e4m3) with per-tensor scales (work-queue and "
                        "indexed workloads); bytes and GB/s count the 1-byte elements")
    p.add_argument("--append", nargs="?", const="separate", choices=("separate", "fused"),
                   help="each step also writes its rows' newest token K/V into the pool: "
                        "'separate' runs append_kv before the op, 'fused' the op's *_append "
                        "variant (the reference harness writes none)")
    p.add_argument("--graph", action="store_true",
                   help="capture the timed steps into one HIP graph and replay it (as the "
                        "reference harness replays captured steps, benchmark_serving_trace.py:1439-1452)")
    p.add_argument("--workspace", choices=("engine", "reference"), default="engine",
                   help="workspace size: this engine's for its faster decomposition, or the "
                        "reference callers' (none for a direct launch)")
    p.add_argument("--cpu-seconds", type=float, default=15.0, help="CPU baseline time budget")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--seed", type=int, default=20260623)
    return p.parse_args()


def cpu_baseline(w, q_pool_cpu, k_cpu, v_cpu, metas, budget_s):
    """Repack + fp32 SDPA on the host for consecutive trace steps until the budget is spent."""
    import torch

    from oracle import attention as oracle

    host_cores = os.cpu_count() or 1
    # The GPU box allots 16 host cores to a one-GPU job (OMP_NUM_THREADS is set to that
    # share there); use them all, and no more than the host has.
    threads = max(1, min(host_cores, int(os.environ.get("OMP_NUM_THREADS", host_cores))))
    torch.set_num_threads(threads)
    tables = [(m.block_table.cpu(), m.seq_lens.cpu(), m.q_indices.cpu(), m.out_indices.cpu())
              for m in metas]

    def step(i):
        if w.op == "attention_contiguous":
            for b in range(len(metas[i].seq_lens)):
                oracle.sdpa_row(q_pool_cpu[i][b], k_cpu[b], v_cpu[b])
        else:
            oracle.paged_decode(q_pool_cpu[i], k_cpu, v_cpu, *tables[i])

    step(0)  # untimed: thread pool and allocator warm-up
    # Consecutive trace steps, the trace repeated, until the budget is spent.
    done_bytes, elapsed, steps = 0, 0.0, 0
    while elapsed < budget_s:
        i = steps % len(metas)
        t0 = time.perf_counter()
        step(i)
        elapsed += time.perf_counter() - t0
        done_bytes += metas[i].kv_bytes
        steps += 1
    if len(metas) == 1:
        what = f"{steps} repeats of the one-step {w.name} trace"
    else:
        passes = f", {steps / len(metas):.1f} passes" if steps > len(metas) else ""
        what = f"{steps} steps of the {len(metas)}-step {w.name} trace{passes}"
    return {"value": round(done_bytes / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "host_cores": host_cores, "cpu_model": cpu_model(),
            "sample": f"{what} ({done_bytes / 1e6:.0f} MB of KV, {elapsed:.1f} s), "
                      f"{elapsed / steps * 1e3:.1f} ms/step, torch CPU SDPA fp32 on {threads} "
                      f"threads"}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def trace_sample(steps, n_trace):
    """Trace step replayed by each timed step: whole passes when ``steps`` is a multiple
    of the trace length, else ``steps`` evenly spaced trace steps."""
    if steps % n_trace == 0:
        return [k % n_trace for k in range(steps)]
    return [(k * n_trace) // steps for k in range(steps)]


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: the engine has no multi-GPU path in this build "
              "(units are independent and would shard by KV head or row); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.steps <= 0:
        print("--steps must be positive", file=sys.stderr)
        sys.exit(2)
    if args.sweep:
        for name in SWEEP:
            result = run_workload(args, name)
            print(json.dumps(result), flush=True)
    else:
        print(json.dumps(run_workload(args, args.workload)), flush=True)


def run_workload(args, workload):
    """Measures one workload and returns its JSON object."""
    import torch

    import persistentkv_torch_ext as ext
    import pkv_serving as serving
    import pkv_workloads as wl

    dev = torch.device("cuda:0")
    w = wl.CONFIGS[workload](seed=args.seed)
    w.fused_merge = args.fused_merge
    w.kv_fp8 = args.kv_fp8
    if w.kv_fp8 and w.op not in ("paged_attention_workqueue", "paged_attention_indexed"):
        print(f"--kv-fp8 applies to the work-queue and indexed workloads, not {w.op}",
              file=sys.stderr)
        sys.exit(2)
    metas = [wl.compile_step(w, i, dev) for i in range(len(w.steps))]
    ws = wl.workspace_for(w, metas, dev, size=args.workspace)
    q_pool = wl.make_q_pool(w, dev)
    wl.bind_queries(metas, q_pool)
    k0, v0 = wl.make_kv_pool(w, dev)
    n_trace = len(w.steps)
    sample = trace_sample(args.steps, n_trace)
    sample_bytes = [metas[i].kv_bytes for i in sample]
    # Enough replicas that the bytes read between two uses of one replica exceed twice the
    # 256 MB Infinity Cache (at most 48 GB of replicas).
    mean_bytes = sum(sample_bytes) / len(sample_bytes)
    pool_bytes = 2 * k0.numel() * k0.element_size()
    rotations = max(args.rotations, -(-2 * MALL_BYTES // int(mean_bytes)) + 1)
    rotations = max(2, min(rotations, int(48e9 // pool_bytes)))
    pools = [(k0, v0)] + [(k0.clone(), v0.clone()) for _ in range(rotations - 1)]
    torch.cuda.synchronize()

    # New-token K/V of every trace step, drawn once and kept on the GPU.
    appends = ([tuple(t.to(dev) for t in wl.new_token_kv(w, i)) for i in range(n_trace)]
               if args.append else None)

    def step(k, i):
        """Timed step k, replaying trace step i."""
        kp, vp = pools[k % len(pools)]
        if args.append == "fused":
            wl.run_step(ext, w, metas[i], i, q_pool, kp, vp, ws, new_kv=appends[i])
            return
        if appends is not None:
            wl.append_step_kv_native(w, i, kp, vp, metas[i], ext, appends[i])
        wl.run_step(ext, w, metas[i], i, q_pool, kp, vp, ws)

    # Correctness gate (reference: benchmark_serving_trace.py:1432-1437), before timing and
    # on a pool nothing has appended to: the middle trace step of the op as timed, against
    # a torch fp32 SDPA over the same pages on the GPU.
    gate_i = n_trace // 2
    if w.kv_fp8:
        gate_k, gate_v = serving.dequantize_pool(k0, w.k_scale), serving.dequantize_pool(v0, w.v_scale)
    elif args.append == "fused":  # the op writes the new token into k0 / v0
        gate_k, gate_v = k0.clone(), v0.clone()
    else:
        gate_k, gate_v = k0, v0
    fused_kv = appends[gate_i] if args.append == "fused" else None
    gate_out = wl.run_step(ext, w, metas[gate_i], gate_i, q_pool, k0, v0, ws, new_kv=fused_kv).clone()
    if fused_kv is not None:  # the reference attends to the appended token too
        serving.append_reference(w, metas[gate_i], gate_k, gate_v, fused_kv)
    torch.cuda.synchronize()
    gate = serving.gate_step(gate_out, metas[gate_i], q_pool[gate_i], gate_k, gate_v, w.page_size)
    gate["step"] = gate_i
    if not gate["pass"]:
        print(f"correctness gate failed at trace step {gate_i} of {workload}: {gate}", file=sys.stderr)
        sys.exit(1)
    del gate_k, gate_v

    graph = None
    if args.graph:
        # Warm up on the capture stream, then capture exactly args.steps steps into one graph.
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for k in range(args.warmup):
                step(k, sample[k % len(sample)])
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for k in range(args.steps):
                    step(k, sample[k])
        torch.cuda.synchronize()
        graph.replay()
    else:
        for k in range(args.warmup):
            step(k, sample[k % len(sample)])
    torch.cuda.synchronize()

    # Timed region: exactly args.steps steps, synchronised on both sides.
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record()
    if graph is not None:
        graph.replay()
    else:
        for k in range(args.steps):
            step(k, sample[k])
    stop.record()
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0
    gpu_ms = start.elapsed_time(stop)
    total_bytes = sum(sample_bytes)

    def decode_stage(i, m, kp, vp):
        # Stage 1 of the op as it runs (the balanced or the per-item schedule).
        ext.paged_attention_workqueue_stage(1, q_pool[i], kp, vp, m.block_table, m.seq_lens,
                                            m.work_items, m.split_offsets, m.q_indices,
                                            m.out_indices, m.output, ws, m.bucket_length,
                                            w.page_size, m.total_partial_slots, w.kv_fp8,
                                            w.k_scale, w.v_scale)

    # Decode kernel alone (stage 1 of the work-queue op) over the same sample, one event
    # pair per launch on its stream.  The grid ops have no separate stage entry point:
    # their whole op is timed.  With the fused merge there are no stages: the op is timed.
    queue = w.op == "paged_attention_workqueue" and not w.fused_merge
    schedule = None
    if w.op == "paged_attention_workqueue":
        schedule = ("balanced" if ext.workqueue_schedule(
            max(len(m.seq_lens) for m in metas), w.hq, w.hkv, w.page_size, ws.numel(),
            w.fused_merge) else "per-item")

    def launch(k):
        i = sample[k]
        kp, vp = pools[k % len(pools)]
        if queue:
            decode_stage(i, metas[i], kp, vp)
        else:
            step(k, i)

    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(args.steps)]
    for k in range(args.steps):
        evs[k][0].record()
        launch(k)
        evs[k][1].record()
    torch.cuda.synchronize()
    dec_ms = [a.elapsed_time(b) for a, b in evs]
    # The same launches back to back under one event pair (no event packets between them).
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b0.record()
    for k in range(args.steps):
        launch(k)
    b1.record()
    torch.cuda.synchronize()
    batched_us = b0.elapsed_time(b1) * 1e3 / args.steps
    merge_us = None
    if queue:
        # Stage 2 (the merge) after its own stage 1, over the same sample: each merge reads
        # the partial states and plan entries its decode wrote.  Launched one by one from
        # Python, a merge of a few microseconds waits on the host's launch rate, so the
        # (decode, merge) pairs and the decodes alone are each replayed from one HIP graph,
        # and the merge's time is the difference.
        def merge_stage(k):
            i = sample[k]
            m = metas[i]
            kp, vp = pools[k % len(pools)]
            ext.paged_attention_workqueue_stage(2, q_pool[i], kp, vp, m.block_table, m.seq_lens,
                                                m.work_items, m.split_offsets, m.q_indices,
                                                m.out_indices, m.output, ws, m.bucket_length,
                                                w.page_size, m.total_partial_slots, w.kv_fp8,
                                                w.k_scale, w.v_scale)

        def graph_us(body):
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            g = torch.cuda.CUDAGraph()
            with torch.cuda.stream(side):
                body()
                with torch.cuda.graph(g, stream=side):
                    body()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) * 1e3 / args.steps

        def pairs():
            for k in range(args.steps):
                launch(k)
                merge_stage(k)

        def decodes():
            for k in range(args.steps):
                launch(k)

        merge_us = graph_us(pairs) - graph_us(decodes)
    # Roofline numerator over the back-to-back launches: event packets between launches
    # add a few microseconds that are not kernel time (rocprofv3's kernel-trace average
    # duration matches the back-to-back figure to about 1 %).
    alg_per_launch = total_bytes / args.steps
    achieved = total_bytes / (batched_us * 1e-6 * args.steps) / 1e9
    traffic, traffic_note = None, None
    traffic_file = TRAFFIC_FILE_FP8 if w.kv_fp8 else TRAFFIC_FILE
    if workload == "c4" and queue and os.path.exists(traffic_file):
        with open(traffic_file) as fh:
            prof = json.load(fh)
        ratio = prof["hbm_bytes_per_launch"] / prof["algorithmic_bytes_per_launch"]
        traffic = int(round(ratio * alg_per_launch))
        traffic_note = (f"rocprofv3 FETCH_SIZE x {prof['fetch_scale']:.2f} + WRITE_SIZE x "
                        f"{prof['write_scale']:.2f} = {ratio:.4f} x algorithmic bytes "
                        f"(profiles/{os.path.basename(traffic_file)}, {prof['launches']} "
                        f"launches), scaled to this sample")

    value = total_bytes / (gpu_ms / 1e3) / 1e9
    published = PUBLISHED_GBPS.get(workload, SWEEP.get(workload))
    kernel = {"paged_attention_workqueue": ("balanced_decode_kernel (stage 1 only)"
                                            if schedule == "balanced" else
                                            "decode_kernel<*,kQueue> (stage 1 only)"),
              "paged_attention_indexed": "decode_kernel<*,kSplit> + merge_kernel (whole op)",
              "paged_attention_masked": "decode_kernel<*,kSplit> + merge_kernel (whole op)",
              "paged_attention": "decode_kernel<*,kDirect> (whole op; split internally into "
                                 "decode_kernel<*,kSplit> + merge_kernel when few units)",
              "attention_contiguous": "decode_kernel<*,kDirect> (whole op; split internally into "
                                      "decode_kernel<*,kSplit> + merge_kernel when few units)"}[w.op]
    if w.op in ("paged_attention", "attention_contiguous") and w.splits > 1:
        kernel = "decode_kernel<*,kSplit> + merge_kernel (whole op)"
    if args.steps % n_trace == 0:
        sample_text = f"{args.steps // n_trace} whole pass(es) of the {n_trace}-step trace"
    else:
        sample_text = f"{args.steps} evenly spaced steps of the {n_trace}-step trace (k * {n_trace} // {args.steps})"
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_s * 1e3 / args.steps, 4),
        "step_us_gpu": round(gpu_ms * 1e3 / args.steps, 2),
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (round(value / published, 3) if published else None),
        "dtype": ("fp16" if w.dtype == torch.float16 else "bf16") + (" (fp8 e4m3 K/V)" if w.kv_fp8 else ""),
        "data": "synthetic",
        "config": {"workload": WORKLOAD_NAMES.get(workload, workload) + ("_fp8kv" if w.kv_fp8 else ""),
                   "requests": len(w.requests),
                   "max_active": max(len(s.active_ids) for s in w.steps),
                   "trace_steps": n_trace, "hq": w.hq, "hkv": w.hkv, "head_dim": 128,
                   "page_size": w.page_size,
                   "splits": "auto (mi355x planner)" if w.auto_splits else w.splits,
                   "fused_merge": bool(args.fused_merge),
                   "schedule": schedule,
                   "launch": "hip graph replay" if args.graph else "eager",
                   "append_kv": args.append or False,
                   "sample": sample_text,
                   "mean_kv_mb_per_step": round(mean_bytes / 1e6, 2),
                   "trace_mean_kv_mb_per_step": round(sum(m.kv_bytes for m in metas) / n_trace / 1e6, 2),
                   "cache_basis": f"HBM-cold ({len(pools)} rotated KV pool replicas)",
                   "workspace_bytes": ws.numel() * ws.element_size(),
                   "workspace": WORKSPACE_LABELS[args.workspace]},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "step_frac": round(value / HBM_PEAK_GBPS, 4),
                     "traffic": traffic,
                     "traffic_source": traffic_note,
                     "kernel": kernel,
                     "mean_launch_us": round(batched_us, 2),
                     "merge_stage_us": None if merge_us is None else round(merge_us, 2),
                     "mean_launch_us_event_bracketed": round(sum(dec_ms) / len(dec_ms) * 1e3, 2),
                     "algorithmic_bytes_per_launch": int(alg_per_launch)},
        "gate": gate,
    }
    if w.op == "attention_contiguous":
        # The reference's query-head baseline on the same inputs (smoke_test.cu:342-374
        # reports the grouped op's speedup over it).
        n_base = max(2, min(args.steps, 16))
        c0, c1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        c0.record()
        for k in range(n_base):
            kp, vp = pools[k % len(pools)]
            ext.attention_query_head_baseline(metas[0].q, kp, vp, metas[0].output)
        c1.record()
        torch.cuda.synchronize()
        base_us = c0.elapsed_time(c1) * 1e3 / n_base
        result["query_head_baseline"] = {"step_us": round(base_us, 2),
                                         "speedup": round(base_us / (gpu_ms * 1e3 / args.steps), 2)}
    if not args.no_cpu_baseline and not args.sweep:
        q_cpu = q_pool.cpu()
        k_cpu, v_cpu = k0.cpu(), v0.cpu()
        if w.kv_fp8:  # the oracle attends to k_scale * e4m3(k8), v_scale * e4m3(v8)
            from oracle import attention as oracle
            k_cpu = oracle.dequantize_e4m3(k_cpu, w.k_scale)
            v_cpu = oracle.dequantize_e4m3(v_cpu, w.v_scale)
        result["cpu_baseline"] = cpu_baseline(w, q_cpu, k_cpu, v_cpu, metas, args.cpu_seconds)
    if published:
        result["published_reference_gbps"] = {
            "value": published, "hardware": "RTX 3060 (360 GB/s)",
            "source": "results/smoke_test.txt (tests/smoke_test.cu bench_perf, contiguous K/V)"}
    return result


if __name__ == "__main__":
    main()
