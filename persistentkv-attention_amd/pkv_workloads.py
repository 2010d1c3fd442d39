"""Serving-trace workloads for the PersistentKV engine (host side of the harness).

Restates the trace mechanics of tests/benchmark_serving_trace.py (rounded_length :159-160,
make_lengths :163-195, build_requests :232-282, build_steps :285-298, make_q_pool
:301-309, the KV pool :1242-1251) and adds the five configurations the engine is
measured on:

  c1  B=1 paged decode, ctx 2048, G=4, fp16, page 16, no split (paged_attention)
  c2  B=8 MHA (G=1), lengths U[1024, 8192], page 16, split 8 (paged_attention_masked)
  c3  B=1 long-context trace, ctx {16384, 32768}, split 32, one token appended to the
      tail page per step (paged_attention_indexed)
  c4  B=8 bimodal continuous-batching trace, 20 work-queue splits (paged_attention_workqueue)
  c5  B=64 Zipf(1.1) lengths, G=32 or 8, bf16, page 32, cost-model splits (work queue)

and the reference's contiguous-layout performance case (smoke_g4_8k, smoke_g4_32k: B=1,
G=4, N 8192 / 32768, 16 splits, attention_contiguous; tests/smoke_test.cu:313-395), with
the whole sweep of that benchmark (SMOKE_SWEEP, :502-521: context, batch and G sweeps) over
contiguous and paged K/V.

Per-step metadata comes from the C++ builder in libpkv.so (pkv_native.build_workqueue);
random values come from torch generators with the reference's seed offsets (pages +99,
Q +2026, KV +7) so that every run of a configuration sees identical inputs.
"""
from __future__ import annotations

import math
from collections import deque
from dataclasses import dataclass, field

import numpy as np
import torch

import pkv_native

HEAD_DIM = 128
DEFAULT_SEED = 20260623  # held-out seed of the reference's review runs


@dataclass(frozen=True)
class Request:
    request_id: int
    arrival: int
    prompt_len: int
    decode_len: int
    physical_pages: tuple


@dataclass(frozen=True)
class StepState:
    step: int
    active_ids: tuple
    lengths: tuple


# ---------------------------------------------------------------------------------
# Reference trace mechanics.
# ---------------------------------------------------------------------------------
def rounded_length(value: int, page_size: int = 16) -> int:
    """benchmark_serving_trace.py:159-160."""
    return max(page_size, ((value + page_size - 1) // page_size) * page_size)


def _randint(gen, lo, hi_inclusive):
    return int(torch.randint(lo, hi_inclusive + 1, (1,), generator=gen).item())


def make_lengths(trace: str, requests: int, seed: int, page_size: int = 16):
    """``[(prompt_len, decode_len)]`` per request; the reference's families
    (benchmark_serving_trace.py:163-195) plus the c3/c4 families of this engine's
    configurations, drawn with the same generator mechanics."""
    gen = torch.Generator(device="cpu")
    gen.manual_seed(seed)
    result = []
    for index in range(requests):
        if trace == "uniform":
            prompt = _randint(gen, 4096, 32768)
            decode = _randint(gen, 16, 96)
        elif trace == "bimodal":
            if index % 4 == 0:
                prompt = _randint(gen, 24576, 65536)
                decode = _randint(gen, 32, 128)
            else:
                prompt = _randint(gen, 2048, 12288)
                decode = _randint(gen, 8, 64)
        elif trace == "zipf":
            rank = _randint(gen, 1, 32)
            prompt = int(2048 + 65536 / math.sqrt(rank))
            jitter = _randint(gen, -512, 512)
            prompt = max(1024, prompt + jitter)
            decode = _randint(gen, 8, 128)
        elif trace == "bucketed":
            prompt = [8192, 16384, 32768, 65536][index % 4]
            decode = _randint(gen, 32, 96)
        elif trace == "homogeneous":
            prompt = 32768
            decode = _randint(gen, 32, 96)
        elif trace == "bimodal_c4":
            # 25 % long rows U[16384, 32768] (every 4th request, as in the reference's
            # bimodal family), 75 % short rows U[256, 1024]; decode lengths as there.
            if index % 4 == 0:
                prompt = _randint(gen, 16384, 32768)
                decode = _randint(gen, 32, 128)
            else:
                prompt = _randint(gen, 256, 1024)
                decode = _randint(gen, 8, 64)
        elif trace == "bucketed_c3":
            prompt = [16384, 32768][index % 2]
            decode = _randint(gen, 32, 96)
        else:
            raise ValueError(f"unknown trace: {trace}")
        result.append((rounded_length(prompt, page_size), decode))
    return result


def load_trace_specs(path, limit, page_size=16):
    """``[(arrival, prompt_len, decode_len)]`` of the first ``limit`` rows of a CSV or JSON
    request trace (benchmark_serving_trace.py:198-229): fields prompt_len (or prompt),
    decode_len (or decode) and optionally arrival (or arrival_step, default the row index);
    prompts rounded up to whole pages."""
    import csv
    import json
    import os
    if os.path.splitext(str(path))[1].lower() == ".json":
        with open(path) as fh:
            rows = json.load(fh)
        if not isinstance(rows, list):
            raise ValueError("a JSON trace file must contain a list of request objects")
    else:
        with open(path, newline="") as fh:
            rows = list(csv.DictReader(fh))
    specs = []
    for index, row in enumerate(rows[:limit]):
        try:
            prompt = int(row.get("prompt_len", row.get("prompt", "")))
            decode = int(row.get("decode_len", row.get("decode", "")))
        except ValueError as error:
            raise ValueError("trace-file rows must define integer prompt_len/prompt and "
                             "decode_len/decode fields") from error
        arrival = int(row.get("arrival", row.get("arrival_step", index)))
        specs.append((arrival, rounded_length(prompt, page_size), decode))
    if not specs:
        raise ValueError(f"trace file produced no requests: {path}")
    return specs


def build_requests(lengths, max_active, seed, hole_fraction, page_size=16, bucket_tokens=0,
                   extra_tokens=0, arrivals=None):
    """Page allocation of benchmark_serving_trace.py:232-282: each request reserves its
    rounded final length in pages; the pool holds ``ceil(total / (1 - holes))`` pages and
    requests take consecutive slices of ``randperm(pool)`` drawn with ``seed + 99``.
    ``extra_tokens`` reserves room for that many tokens beyond prompt + decode; request i
    arrives at ``arrivals[i]`` (a trace file's) or ``i // max_active``."""
    logical = []
    for prompt, decode in lengths:
        exact = prompt + decode + extra_tokens
        if bucket_tokens > 0:
            reserved = rounded_length(((exact + bucket_tokens - 1) // bucket_tokens) * bucket_tokens,
                                      page_size)
        else:
            reserved = rounded_length(exact, page_size)
        logical.append(math.ceil(reserved / page_size))
    total = sum(logical)
    physical_pages = math.ceil(total / max(1e-6, 1.0 - hole_fraction))
    ids = torch.randperm(physical_pages, generator=torch.Generator().manual_seed(seed + 99))
    built, cursor = [], 0
    for request_id, ((prompt, decode), pages) in enumerate(zip(lengths, logical)):
        assigned = tuple(int(x) for x in ids[cursor:cursor + pages].tolist())
        cursor += pages
        arrival = arrivals[request_id] if arrivals is not None else request_id // max_active
        built.append(Request(request_id, arrival, prompt, decode, assigned))
    return built, physical_pages


def build_steps(requests, max_active):
    """Reference admission rule (benchmark_serving_trace.py:285-298): request i arrives at
    ``i // max_active`` and ages from then on; each step serves the first ``max_active``
    requests (by id) that are within their decode window."""
    steps = []
    max_step = max(req.arrival + req.decode_len for req in requests)
    for step in range(max_step):
        candidates = []
        for req in requests:
            generated = step - req.arrival
            if 0 <= generated < req.decode_len:
                candidates.append((req.request_id, req.prompt_len + generated))
        candidates = candidates[:max_active]
        if candidates:
            active_ids, lengths = zip(*candidates)
            steps.append(StepState(step, tuple(active_ids), tuple(lengths)))
    return steps


def build_steps_continuous(requests, max_active, max_steps):
    """Continuous batching: every request is waiting at step 0; up to ``max_active`` are
    served per step; a request retires after ``decode_len`` tokens and the next waiting
    request is admitted at the following step."""
    waiting = deque(requests)
    active, generated, steps = [], {}, []
    for step in range(max_steps):
        while len(active) < max_active and waiting:
            req = waiting.popleft()
            active.append(req)
            generated[req.request_id] = 0
        if not active:
            break
        steps.append(StepState(step, tuple(r.request_id for r in active),
                               tuple(r.prompt_len + generated[r.request_id] for r in active)))
        for r in active:
            generated[r.request_id] += 1
        active = [r for r in active if generated[r.request_id] < r.decode_len]
    return steps


def zipf_lengths(count, seed, s=1.1, lo=128, hi=65536):
    """``count`` lengths with P(L) proportional to L^-s on [lo, hi] (inverse CDF with a
    float64 torch uniform drawn from ``seed``)."""
    support = np.arange(lo, hi + 1, dtype=np.float64)
    cdf = np.cumsum(support ** (-s))
    cdf /= cdf[-1]
    gen = torch.Generator().manual_seed(seed)
    u = torch.rand(count, generator=gen, dtype=torch.float64).numpy()
    return [int(support[min(int(np.searchsorted(cdf, x)), len(support) - 1)]) for x in u]


# ---------------------------------------------------------------------------------
# Configurations.
# ---------------------------------------------------------------------------------
@dataclass
class Workload:
    name: str
    op: str                 # paged_attention | paged_attention_masked | _indexed | _workqueue
                            # | attention_contiguous
    hq: int
    hkv: int
    page_size: int
    dtype: torch.dtype
    seed: int
    requests: list
    steps: list
    physical_pages: int
    splits: int = 1
    auto_splits: bool = False
    policy: int = pkv_native.POLICY_REFERENCE
    append_kv: bool = False
    fused_merge: bool = False
    # fp8 (OCP e4m3) K/V pages with per-tensor scales (indexed and work-queue ops only).
    kv_fp8: bool = False
    k_scale: float = 1.0 / 64.0
    v_scale: float = 1.0 / 64.0
    extra: dict = field(default_factory=dict)

    @property
    def group(self):
        return self.hq // self.hkv

    def kv_bytes(self, step_index):
        """Algorithmic K+V bytes of one decode step:
        sum(lengths) * Hkv * 128 * 2 (K and V) * element bytes (the reference's
        useful_kv_mb_for_state, benchmark_serving_trace.py:511-513, in bytes)."""
        elem = 1 if self.kv_fp8 else 2
        return sum(self.steps[step_index].lengths) * self.hkv * HEAD_DIM * 2 * elem


def config_c1(seed=DEFAULT_SEED):
    """B=1, Hq 32 / Hkv 8, ctx 2048, page 16, 128 pages drawn from a 4096-page pool."""
    gen = torch.Generator().manual_seed(seed + 99)
    pages = tuple(int(x) for x in torch.randperm(4096, generator=gen)[:128].tolist())
    req = Request(0, 0, 2048, 1, pages)
    return Workload("c1", "paged_attention", 32, 8, 16, torch.float16, seed, [req],
                    [StepState(0, (0,), (2048,))], 4096, splits=1)


def config_c2(seed=DEFAULT_SEED):
    """B=8 MHA (Hq = Hkv = 32), lengths U[1024, 8192], pool 1.5x the used pages, split 8."""
    gen = torch.Generator().manual_seed(seed)
    lengths = [int(x) for x in torch.randint(1024, 8193, (8,), generator=gen).tolist()]
    pages = [math.ceil(n / 16) for n in lengths]
    physical = math.ceil(1.5 * sum(pages))
    ids = torch.randperm(physical, generator=torch.Generator().manual_seed(seed + 99))
    reqs, cursor = [], 0
    for i, (n, p) in enumerate(zip(lengths, pages)):
        reqs.append(Request(i, 0, n, 1, tuple(int(x) for x in ids[cursor:cursor + p].tolist())))
        cursor += p
    return Workload("c2", "paged_attention_masked", 32, 32, 16, torch.float16, seed, reqs,
                    [StepState(0, tuple(range(8)), tuple(lengths))], physical, splits=8)


def config_c3(seed=DEFAULT_SEED, steps=64, first_bucket=16384):
    """B=1 long-context trace: 16 requests with prompts alternating 16384 / 32768 served one
    at a time, 64 steps, split 32, each step appending one token's K/V.  With
    ``first_bucket=32768`` the alternation starts at the 32k bucket (the B1 32k-context
    case; the 16k-first trace spends its 64 steps in the first request)."""
    lengths = make_lengths("bucketed_c3", 16, seed)
    if first_bucket == 32768:
        lengths = [(lengths[i ^ 1][0], lengths[i][1]) for i in range(len(lengths))]
    reqs, physical = build_requests(lengths, 1, seed, 0.0)
    st = build_steps_continuous(reqs, 1, steps)
    name = "c3" if first_bucket == 16384 else "c3_32k"
    return Workload(name, "paged_attention_indexed", 32, 8, 16, torch.float16, seed, reqs, st,
                    physical, splits=32, append_kv=True)


def config_c4(seed=DEFAULT_SEED, steps=48, fused_merge=False):
    """B=8 bimodal continuous batching: 24 requests (every 4th long, U[16384, 32768];
    others U[256, 1024]), max-active 8, 48 steps, 20 fixed work-queue splits."""
    lengths = make_lengths("bimodal_c4", 24, seed)
    reqs, physical = build_requests(lengths, 8, seed, 0.0)
    st = build_steps_continuous(reqs, 8, steps)
    return Workload("c4", "paged_attention_workqueue", 32, 8, 16, torch.float16, seed, reqs, st,
                    physical, splits=20, fused_merge=fused_merge)


def config_c5(hkv=1, seed=DEFAULT_SEED, steps=48, batch=64):
    """B=64 Zipf(1.1) lengths in [128, 65536], Hq 32 with Hkv 1 (G=32) or 4 (G=8), bf16,
    page 32, 10 % free-page holes, 48 steps, work queue with the MI355X split planner."""
    prompts = zipf_lengths(batch, seed)
    lengths = [(rounded_length(p, 32), steps) for p in prompts]
    reqs, physical = build_requests(lengths, batch, seed, 0.10, page_size=32)
    reqs = [Request(r.request_id, 0, r.prompt_len, r.decode_len, r.physical_pages) for r in reqs]
    st = build_steps(reqs, batch)[:steps]
    return Workload(f"c5_g{32 // hkv}", "paged_attention_workqueue", 32, hkv, 32, torch.bfloat16,
                    seed, reqs, st, physical, splits=1, auto_splits=True,
                    policy=pkv_native.POLICY_MI355X)


def config_smoke(context, seed=DEFAULT_SEED, batch=1, hq=32, hkv=8, splits=16):
    """The reference's contiguous-layout performance case (tests/smoke_test.cu bench_perf,
    :313-395): K/V ``[B, Hkv, N, 128]`` fp16, B=1, Hq 32 / Hkv 8, 16 splits, published at
    N = 8192 and 32768 (results/smoke_test.txt:25, :27).  Each row owns one "page" of N
    tokens: the slab ``[row]`` of K and V."""
    reqs = [Request(i, 0, context, 1, (i,)) for i in range(batch)]
    step = StepState(0, tuple(range(batch)), (context,) * batch)
    return Workload(f"smoke_g{hq // hkv}_{context // 1024}k", "attention_contiguous", hq, hkv,
                    context, torch.float16, seed, reqs, [step], batch, splits=splits)


def config_trace(trace="bimodal", requests=24, max_active=8, steps=48, seed=20260622,
                 hole_fraction=0.50, page_size=16, hkv=8, hq=32, splits=16, bucket_tokens=0,
                 trace_file=None):
    """A trace of the reference's serving harness with its command-line options and
    defaults (benchmark_serving_trace.py:1114-1163; main :1219-1229): the request family
    (make_lengths) or a trace file, the page allocation with the hole fraction and bucket
    rounding (build_requests), the reference's admission rule (build_steps) cut to
    ``steps``, fp16, Hq 32.  Run through the work-queue op with ``splits``."""
    if trace_file is not None:
        specs = load_trace_specs(trace_file, requests, page_size)
        lengths = [(p, d) for _, p, d in specs]
        arrivals = [a for a, _, _ in specs]
    else:
        lengths = make_lengths(trace, requests, seed, page_size)
        arrivals = None
    reqs, physical = build_requests(lengths, max_active, seed, hole_fraction, page_size,
                                    bucket_tokens, arrivals=arrivals)
    st = build_steps(reqs, max_active)[:steps]
    if not st:
        raise ValueError("the trace produced no active decode steps")
    name = "trace_file" if trace_file is not None else f"trace_{trace}"
    return Workload(name, "paged_attention_workqueue", hq, hkv, page_size, torch.float16, seed,
                    reqs, st, physical, splits=splits,
                    extra={"trace": trace, "max_active": max_active, "hole_fraction": hole_fraction,
                           "bucket_tokens": bucket_tokens, "trace_file": trace_file})


def config_smoke_paged(context, seed=DEFAULT_SEED, batch=1, hq=32, hkv=8, splits=16, page_size=16):
    """config_smoke over a paged pool: each of the B rows holds N tokens in pages of
    ``page_size`` drawn by a seeded permutation of a pool 1.5x the used pages, run through
    ``paged_attention`` (every row attends to N tokens) with the same split count."""
    pages = -(-context // page_size)
    physical = math.ceil(1.5 * pages * batch)
    ids = torch.randperm(physical, generator=torch.Generator().manual_seed(seed + 99)).tolist()
    reqs = [Request(i, 0, context, 1, tuple(int(x) for x in ids[i * pages:(i + 1) * pages]))
            for i in range(batch)]
    step = StepState(0, tuple(range(batch)), (context,) * batch)
    return Workload(f"smoke_g{hq // hkv}_{context // 1024}k_paged", "paged_attention", hq, hkv,
                    page_size, torch.float16, seed, reqs, [step], physical, splits=splits)


# The reference's performance sweep (tests/smoke_test.cu:502-521, contiguous K/V through
# persistentkv_split_dispatch) with its published bandwidth on an RTX 3060
# (results/smoke_test.txt:23-43): (B, Hq, Hkv, N, splits, GB/s).
SMOKE_SWEEP = [
    (1, 32, 8, 4096, 16, 221.9), (1, 32, 8, 8192, 16, 237.1), (1, 32, 8, 16384, 16, 236.3),
    (1, 32, 8, 32768, 16, 238.6),                                  # GQA, G = 4
    (1, 8, 1, 4096, 128, 33.4), (1, 8, 1, 8192, 128, 47.0),        # MQA-like, G = 8
    (1, 32, 8, 8192, 16, 237.4), (2, 32, 8, 8192, 8, 247.0), (4, 32, 8, 8192, 4, 241.7),
    (8, 32, 8, 8192, 2, 229.5),                                    # batch sweep
    (1, 4, 4, 8192, 32, 101.7), (1, 8, 4, 8192, 32, 100.0), (1, 16, 4, 8192, 32, 196.3),
    (1, 32, 4, 8192, 32, 55.2),                                    # G sweep (1, 2, 4, 8)
]


def sweep_name(b, hq, hkv, n, splits, paged=False):
    return f"sweep_b{b}_hq{hq}_hkv{hkv}_n{n}_s{splits}" + ("_paged" if paged else "")


def sweep_configs():
    """Workload factories of SMOKE_SWEEP, contiguous and paged, by name."""
    out = {}
    for b, hq, hkv, n, splits, _ in SMOKE_SWEEP:
        for paged in (False, True):
            make = config_smoke_paged if paged else config_smoke
            out[sweep_name(b, hq, hkv, n, splits, paged)] = (
                lambda make=make, b=b, hq=hq, hkv=hkv, n=n, s=splits, **kw:
                make(n, batch=b, hq=hq, hkv=hkv, splits=s, **kw))
    return out


CONFIGS = {"c1": config_c1, "c2": config_c2, "c3": config_c3,
           "c3_32k": lambda **kw: config_c3(first_bucket=32768, **kw), "c4": config_c4,
           "c5_g32": lambda **kw: config_c5(hkv=1, **kw), "c5_g8": lambda **kw: config_c5(hkv=4, **kw),
           "smoke_g4_8k": lambda **kw: config_smoke(8192, **kw),
           "smoke_g4_32k": lambda **kw: config_smoke(32768, **kw),
           **sweep_configs()}


# ---------------------------------------------------------------------------------
# Device state and per-step metadata.
# ---------------------------------------------------------------------------------
def make_kv_pool(w: Workload, device, seed_offset=7):
    """K and V pools ``[pages, Hkv, page_size, 128]`` ~ N(0, 1) (reference :1242-1251).
    For the contiguous op a page is one row's N tokens, so this is ``[B, Hkv, N, 128]``."""
    gen = torch.Generator(device=device)
    gen.manual_seed(w.seed + seed_offset)
    shape = (w.physical_pages, w.hkv, w.page_size, HEAD_DIM)
    k = torch.randn(*shape, generator=gen, device=device, dtype=w.dtype)
    v = torch.randn(*shape, generator=gen, device=device, dtype=w.dtype)
    if w.kv_fp8:  # N(0, 1) values quantised with the workload's per-tensor scales
        k = (k.float() / w.k_scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        v = (v.float() / w.v_scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return k, v


def make_q_pool(w: Workload, device):
    """Q ``[steps, requests, Hq, 128]`` ~ N(0, 1) drawn on the CPU with ``seed + 2026``
    (reference :301-309), then moved to ``device``."""
    gen = torch.Generator().manual_seed(w.seed + 2026)
    q = torch.randn(len(w.steps), len(w.requests), w.hq, HEAD_DIM, generator=gen,
                    dtype=torch.float32)
    return q.to(w.dtype).to(device)


@dataclass
class StepMeta:
    op: str
    bucket_length: int
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    q_indices: torch.Tensor
    out_indices: torch.Tensor
    output: torch.Tensor
    splits: int
    work_items: torch.Tensor | None = None
    split_offsets: torch.Tensor | None = None
    merge_counters: torch.Tensor | None = None
    total_partial_slots: int = 0
    num_tasks: int = 0
    kv_bytes: int = 0
    q: torch.Tensor | None = None  # gathered query rows for the ops without q_indices


def compile_step(w: Workload, step_index: int, device) -> StepMeta:
    """Block table, lengths, indices and (work-queue op) the compact work queue of one
    step, built on the host by libpkv.so and copied to ``device``."""
    st = w.steps[step_index]
    by_id = {r.request_id: r for r in w.requests}
    page_lists = [by_id[i].physical_pages for i in st.active_ids]
    t = lambda a: torch.as_tensor(np.ascontiguousarray(a), dtype=torch.int32).to(device)
    n = len(st.active_ids)
    output = torch.empty(n, w.hq, HEAD_DIM, device=device, dtype=w.dtype)
    if w.op == "paged_attention_workqueue":
        meta = pkv_native.build_workqueue(list(st.lengths), list(st.active_ids), page_lists,
                                          w.page_size, w.splits, w.auto_splits, w.hkv, w.policy,
                                          hq=w.hq)
        return StepMeta(w.op, meta["bucket_length"], t(meta["block_table"]), t(meta["seq_lens"]),
                        t(meta["q_indices"]), t(meta["out_indices"]), output, meta["splits"],
                        t(meta["work_items"]), t(meta["split_offsets"]),
                        torch.zeros(n, w.hkv, device=device, dtype=torch.int32),
                        meta["total_partial_slots"], int(meta["work_items"].shape[0]),
                        w.kv_bytes(step_index))
    bucket = max(st.lengths)
    cols = math.ceil(bucket / w.page_size)
    table = np.array([list(p[:cols]) + [p[-1]] * (cols - len(p[:cols])) for p in page_lists],
                     dtype=np.int32)
    return StepMeta(w.op, bucket, t(table), t(np.array(st.lengths)), t(np.array(st.active_ids)),
                    t(np.arange(n)), output, w.splits, kv_bytes=w.kv_bytes(step_index))


def workspace_for(w: Workload, metas, device, balanced=True, size="engine"):
    """One fp32 workspace for every step of ``metas``.

    ``size="engine"``: the work queue's partial states (and, with ``balanced``, at least
    what its balanced schedule needs, pkv_workqueue_balanced_workspace_bytes), a split
    grid's with room for its internal sub-split (pkv_split_workspace_bytes), or for a
    direct (num_splits == 1) launch the size at which the op runs its full internal split
    (pkv_direct_workspace_bytes).
    ``size="reference"``: the sizes the reference's callers allocate, which the op must
    also accept: ``total_partial_slots * Hq * 130`` floats for the work queue,
    ``B * Hq * S * 130`` for a split grid and none for a direct launch."""
    if size not in ("engine", "reference"):
        raise ValueError(f"workspace size must be 'engine' or 'reference', not {size!r}")
    floats = 0
    for m in metas:
        if m.op == "paged_attention_workqueue":
            floats = max(floats, m.total_partial_slots * w.hq * (2 + HEAD_DIM))
            if balanced and size == "engine":
                floats = max(floats, pkv_native.workqueue_balanced_workspace_bytes(
                    len(m.seq_lens), w.hq, w.hkv) // 4)
        elif size == "reference":
            if m.splits > 1:
                floats = max(floats, len(m.seq_lens) * w.hq * m.splits * (2 + HEAD_DIM))
        elif m.splits > 1:
            floats = max(floats, pkv_native.split_workspace_bytes(
                len(m.seq_lens), w.hq, w.hkv, m.bucket_length, m.splits) // 4)
        else:
            floats = max(floats, pkv_native.direct_workspace_bytes(
                len(m.seq_lens), w.hq, w.hkv, m.bucket_length) // 4)
    if size == "engine":
        floats = max(floats, 1)
    return torch.empty(floats, device=device, dtype=torch.float32)


def bind_queries(metas, q_pool):
    """Gathers, once, the query rows of each step for the two ops that take Q already in
    row order (``paged_attention``, ``paged_attention_masked``), so that a timed step runs
    only the op itself."""
    for i, m in enumerate(metas):
        if m.op in ("paged_attention", "paged_attention_masked", "attention_contiguous"):
            m.q = q_pool[i].index_select(0, m.q_indices.long()).contiguous()
    return metas


def run_step(ext, w: Workload, meta: StepMeta, step_index: int, q_pool, k_pages, v_pages,
             workspace, new_kv=None):
    """One decode step through the op the workload names; returns ``meta.output``.
    ``new_kv`` = (k_new, v_new) of the step's rows runs the op's *_append variant, which
    also writes them into the pools (indexed and work-queue ops)."""
    q_source = q_pool[step_index]
    if new_kv is not None:
        if meta.op not in ("paged_attention_workqueue", "paged_attention_indexed",
                           "paged_attention_masked"):
            raise ValueError(f"the fused append is provided for the work-queue, indexed and "
                             f"masked ops, not {meta.op}")
        if meta.op == "paged_attention_masked" and w.kv_fp8:
            raise ValueError("the masked op has no fp8 variant")
        if meta.op == "paged_attention_workqueue" and w.kv_fp8:
            ext.paged_attention_workqueue_fp8_append(
                q_source, k_pages, v_pages, meta.block_table, meta.seq_lens, meta.work_items,
                meta.split_offsets, meta.merge_counters, meta.q_indices, meta.out_indices,
                meta.output, workspace, meta.bucket_length, w.page_size, meta.total_partial_slots,
                w.fused_merge, w.k_scale, w.v_scale, new_kv[0], new_kv[1])
        elif meta.op == "paged_attention_indexed" and w.kv_fp8:
            ext.paged_attention_indexed_fp8_append(
                q_source, k_pages, v_pages, meta.block_table, meta.seq_lens, meta.q_indices,
                meta.out_indices, meta.output, workspace, meta.bucket_length, w.page_size,
                meta.splits, w.k_scale, w.v_scale, new_kv[0], new_kv[1])
        elif meta.op == "paged_attention_workqueue":
            ext.paged_attention_workqueue_append(
                q_source, k_pages, v_pages, meta.block_table, meta.seq_lens, meta.work_items,
                meta.split_offsets, meta.merge_counters, meta.q_indices, meta.out_indices,
                meta.output, workspace, meta.bucket_length, w.page_size, meta.total_partial_slots,
                w.fused_merge, new_kv[0], new_kv[1])
        elif meta.op == "paged_attention_masked":
            q = meta.q if meta.q is not None else q_source.index_select(0, meta.q_indices.long()).contiguous()
            ext.paged_attention_masked_append(
                q, k_pages, v_pages, meta.block_table, meta.seq_lens, meta.output, workspace,
                meta.bucket_length, w.page_size, meta.splits, new_kv[0], new_kv[1])
        else:
            ext.paged_attention_indexed_append(
                q_source, k_pages, v_pages, meta.block_table, meta.seq_lens, meta.q_indices,
                meta.out_indices, meta.output, workspace, meta.bucket_length, w.page_size,
                meta.splits, new_kv[0], new_kv[1])
        return meta.output
    if w.kv_fp8 and meta.op not in ("paged_attention_workqueue", "paged_attention_indexed"):
        raise ValueError(f"fp8 K/V is provided for the work-queue and indexed ops, not {meta.op}")
    if meta.op == "paged_attention_workqueue" and w.kv_fp8:
        ext.paged_attention_workqueue_fp8(q_source, k_pages, v_pages, meta.block_table,
                                          meta.seq_lens, meta.work_items, meta.split_offsets,
                                          meta.merge_counters, meta.q_indices, meta.out_indices,
                                          meta.output, workspace, meta.bucket_length, w.page_size,
                                          meta.total_partial_slots, w.fused_merge, w.k_scale,
                                          w.v_scale)
    elif meta.op == "paged_attention_workqueue":
        ext.paged_attention_workqueue(q_source, k_pages, v_pages, meta.block_table, meta.seq_lens,
                                      meta.work_items, meta.split_offsets, meta.merge_counters,
                                      meta.q_indices, meta.out_indices, meta.output, workspace,
                                      meta.bucket_length, w.page_size, meta.total_partial_slots,
                                      w.fused_merge)
    elif meta.op == "paged_attention_indexed" and w.kv_fp8:
        ext.paged_attention_indexed_fp8(q_source, k_pages, v_pages, meta.block_table,
                                        meta.seq_lens, meta.q_indices, meta.out_indices,
                                        meta.output, workspace, meta.bucket_length, w.page_size,
                                        meta.splits, w.k_scale, w.v_scale)
    elif meta.op == "paged_attention_indexed":
        ext.paged_attention_indexed(q_source, k_pages, v_pages, meta.block_table, meta.seq_lens,
                                    meta.q_indices, meta.out_indices, meta.output, workspace,
                                    meta.bucket_length, w.page_size, meta.splits)
    elif meta.op == "paged_attention_masked":
        q = meta.q if meta.q is not None else q_source.index_select(0, meta.q_indices.long()).contiguous()
        ext.paged_attention_masked(q, k_pages, v_pages, meta.block_table, meta.seq_lens,
                                   meta.output, workspace, meta.bucket_length, w.page_size,
                                   meta.splits)
    elif meta.op == "attention_contiguous":
        q = meta.q if meta.q is not None else q_source.index_select(0, meta.q_indices.long()).contiguous()
        ext.attention_contiguous(q, k_pages, v_pages, meta.output, workspace, meta.splits)
    elif meta.op == "paged_attention":
        q = meta.q if meta.q is not None else q_source.index_select(0, meta.q_indices.long()).contiguous()
        ext.paged_attention(q, k_pages, v_pages, meta.block_table, meta.output, workspace,
                            meta.bucket_length, w.page_size, meta.splits)
    else:
        raise ValueError(meta.op)
    return meta.output


def new_token_kv(w: Workload, step_index: int, seed_offset=11):
    """K and V ``[active rows, Hkv, 128]`` of each active row's newest token at a step,
    drawn on the CPU from ``seed + seed_offset + step`` (row by row, K then V), in the
    workload's dtype."""
    st = w.steps[step_index]
    gen = torch.Generator().manual_seed(w.seed + seed_offset + step_index)
    ks, vs = [], []
    for _ in st.active_ids:
        ks.append(torch.randn(w.hkv, HEAD_DIM, generator=gen).to(w.dtype))
        vs.append(torch.randn(w.hkv, HEAD_DIM, generator=gen).to(w.dtype))
    return torch.stack(ks), torch.stack(vs)


def append_step_kv_native(w: Workload, step_index: int, k_pages, v_pages, meta, ext,
                          new_kv=None, seed_offset=11):
    """append_step_kv on the GPU: one ``append_kv`` (``append_kv_fp8`` for fp8 pools)
    launch over the step's rows, using the step's compiled block table and lengths.
    ``new_kv`` is the step's (K, V) already on the device (new_token_kv otherwise)."""
    if new_kv is None:
        new_kv = tuple(t.to(k_pages.device) for t in new_token_kv(w, step_index, seed_offset))
    k_new, v_new = new_kv
    if w.kv_fp8:
        ext.append_kv_fp8(k_new, v_new, k_pages, v_pages, meta.block_table, meta.seq_lens,
                          w.k_scale, w.v_scale)
    else:
        ext.append_kv(k_new, v_new, k_pages, v_pages, meta.block_table, meta.seq_lens)


def append_step_kv(w: Workload, step_index: int, k_pages, v_pages, seed_offset=11):
    """Writes the K/V of each active row's newest token (position length - 1) into its
    tail page, with values drawn from ``seed + seed_offset + step``: the host-side
    restatement of append_step_kv_native (one indexed write per row)."""
    st = w.steps[step_index]
    by_id = {r.request_id: r for r in w.requests}
    gen = torch.Generator().manual_seed(w.seed + seed_offset + step_index)
    for rid, length in zip(st.active_ids, st.lengths):
        pos = length - 1
        page = by_id[rid].physical_pages[pos // w.page_size]
        k_new = torch.randn(w.hkv, HEAD_DIM, generator=gen).to(w.dtype)
        v_new = torch.randn(w.hkv, HEAD_DIM, generator=gen).to(w.dtype)
        if w.kv_fp8:
            k_new = (k_new.float() / w.k_scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
            v_new = (v_new.float() / w.v_scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
        k_pages[page, :, pos % w.page_size] = k_new.to(k_pages.device)
        v_pages[page, :, pos % w.page_size] = v_new.to(v_pages.device)
