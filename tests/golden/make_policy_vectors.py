"""Writes tests/golden/policy_vectors.json from the reference's own host functions.

Run in the build container only (the reference is not present on GPU machines):

    python tests/golden/make_policy_vectors.py /root/reference

It imports tests/benchmark_serving_trace.py of ahmed123hds/persistentkv-attention and
records input/output pairs of its CPU-only functions, which no closed form pins:
  * split policies  choose_splits :328-367, choose_workqueue_row_splits :370-393,
                    model_bucket_splits :396-402, model_workqueue_splits :405-415
  * cost model      estimate_route_ms :418-442, choose_adaptive_route_cost_model :445-488
  * trace RNG       make_lengths :163-195, build_requests :232-282, build_steps :285-298
  * length buckets  round_bucket_length :316-321, use_single_bucket_for_state :491-504
The module globals HKV and PAGE_SIZE are set the way the reference's main() sets them
(:1215-1217).  Functions that touch the GPU are not called.  The draws of each section
come after those of the sections above it, so adding a section leaves the earlier
vectors unchanged.
"""
from __future__ import annotations

import importlib.util
import json
import os
import random
import struct
import sys
import zlib

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference(root):
    path = os.path.join(root, "tests", "benchmark_serving_trace.py")
    spec = importlib.util.spec_from_file_location("reference_serving_trace", path)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod  # dataclasses resolve their module through sys.modules
    spec.loader.exec_module(mod)
    return mod


def main(root):
    ref = load_reference(root)
    rng = random.Random(1234)
    out = {"source": "tests/benchmark_serving_trace.py", "row_splits": [], "choose_splits": [],
           "model_splits": [], "routes": [], "traces": [], "round_bucket": [],
           "single_bucket": []}

    lengths_grid = [0, 1, 31, 32, 33, 100, 255, 256, 511, 512, 1023, 1024, 2047, 2048, 4096,
                    6000, 8192, 12288, 16383, 16384, 16385, 24576, 32768, 49152, 65536, 131072]
    active_grid = [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16, 32, 64]
    for hkv in (1, 4, 8, 16, 32):
        ref.HKV = hkv
        for length in lengths_grid:
            for active in active_grid:
                for req, auto in ((20, False), (1, True)):
                    out["row_splits"].append(
                        [hkv, length, active, req, int(auto),
                         ref.choose_workqueue_row_splits(length, active, req, auto)])

    def random_lengths(n):
        kind = rng.random()
        if kind < 0.3:
            return [rng.randint(1, 2048) for _ in range(n)]
        if kind < 0.6:
            return [rng.randint(256, 70000) for _ in range(n)]
        return [rng.choice([256, 1024, 8192, 16384, 32768, 65536]) + rng.randint(0, 96)
                for _ in range(n)]

    for hkv in (4, 8, 32):
        ref.HKV = hkv
        for _ in range(300):
            n = rng.choice([1, 2, 3, 4, 5, 7, 8, 9, 16])
            lens = random_lengths(n)
            for single in (False, True):
                out["choose_splits"].append(
                    [hkv, lens, int(single), ref.choose_splits(lens, 16, True, single)])
            state = ref.StepState(0, tuple(range(n)), tuple(lens))
            out["model_splits"].append([hkv, lens, ref.model_bucket_splits(state),
                                        ref.model_workqueue_splits(state)])

    for hkv in (4, 8, 16):
        ref.HKV = hkv
        for _ in range(200):
            n = rng.choice([1, 1, 2, 4, 8, 8, 12])
            lens = random_lengths(n)
            state = ref.StepState(0, tuple(range(n)), tuple(lens))
            est = {route: [[s, ref.estimate_route_ms(state, route, s)] for s in (1, 4, 16, 20, 48)]
                   for route in ("flashinfer", "persistentkv_bucket", "persistentkv_workqueue")}
            choice = ref.choose_adaptive_route_cost_model(state)
            out["routes"].append([hkv, lens, est, [choice.route, choice.splits, choice.estimated_ms]])

    ref.HKV = 8
    for trace in ("uniform", "bimodal", "zipf", "bucketed", "homogeneous"):
        for seed, requests, max_active, holes, page in ((20260622, 12, 4, 0.5, 16),
                                                        (20260623, 24, 8, 0.0, 16),
                                                        (7, 9, 3, 0.25, 32)):
            ref.PAGE_SIZE = page
            lengths = ref.make_lengths(trace, requests, seed)
            reqs, physical = ref.build_requests(trace, requests, max_active, seed, holes, 0, None)
            steps = ref.build_steps(reqs, max_active)
            out["traces"].append({
                "trace": trace, "seed": seed, "requests": requests, "max_active": max_active,
                "hole_fraction": holes, "page_size": page, "lengths": lengths,
                "physical_pages": physical,
                # page lists as (count, first 4 ids, crc32 of the int32 little-endian ids)
                "pages": [[len(r.physical_pages), list(r.physical_pages[:4]),
                           zlib.crc32(struct.pack(f"<{len(r.physical_pages)}i", *r.physical_pages))]
                          for r in reqs],
                "arrivals": [r.arrival for r in reqs],
                "steps": [[s.step, list(s.active_ids), list(s.lengths)] for s in steps],
            })
    ref.PAGE_SIZE = 16

    # round_bucket_length(length, bucket_tokens, allocated_pages) at each page size.
    for page in (8, 16, 32, 64, 128):
        ref.PAGE_SIZE = page
        for length in (1, 7, 8, 15, 16, 17, 100, 1000, 1024, 4095, 4096, 4097, 16384, 20000,
                       32768, 65535, 65536):
            for bucket_tokens in (-1, 0, 1, 16, 100, 512, 1024, 4096, 8192):
                for pages in (0, 1, 3, 64, 512, 5000):
                    out["round_bucket"].append(
                        [page, length, bucket_tokens, pages,
                         ref.round_bucket_length(length, bucket_tokens, pages)])
    ref.PAGE_SIZE = 16
    # use_single_bucket_for_state(state, requested_single_bucket, adaptive_route).
    for _ in range(400):
        n = rng.choice([1, 2, 3, 4, 5, 6, 8, 9, 16])
        pool = rng.choice([[1024], [1024, 2048], [100, 200, 300, 400], list(range(1, 40))])
        lens = [rng.choice(pool) for _ in range(n)]
        state = ref.StepState(0, tuple(range(n)), tuple(lens))
        for single in (False, True):
            for adaptive in (False, True):
                out["single_bucket"].append(
                    [lens, int(single), int(adaptive),
                     int(ref.use_single_bucket_for_state(state, single, adaptive))])

    path = os.path.join(HERE, "policy_vectors.json")
    with open(path, "w") as fh:
        json.dump(out, fh, separators=(",", ":"))
    print(f"wrote {path}: " + ", ".join(f"{k}={len(v)}" for k, v in out.items() if isinstance(v, list)))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
