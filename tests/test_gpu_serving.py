"""The serving harness on the GPU: multi-bucket steps through per-bucket
paged_attention_indexed launches (the reference's length-bucket route,
benchmark_serving_trace.py:731-780, :986-1000) and the adaptive engine's routed steps,
each against the repack + fp32 SDPA oracle; and the harness's own gate."""
import pytest
import torch

import pkv_serving as serving
import pkv_workloads as wl
from oracle import attention as oracle
from paged_cases import assert_parity

pytestmark = pytest.mark.gpu


def _oracle(w, meta, q_source, k_pages, v_pages):
    """Oracle output [rows, Hq, 128] (rows in output order); only each row's pages leave
    the GPU."""
    out = torch.zeros(meta.output.shape[0], w.hq, 128)
    for b, n in enumerate(meta.seq_lens.tolist()):
        pages = meta.block_table[b, : -(-n // w.page_size)].long()
        k = k_pages.index_select(0, pages).cpu()
        v = v_pages.index_select(0, pages).cpu()
        kk, vv = oracle.gather_row(k, v, torch.arange(len(pages), dtype=torch.int32), n)
        out[int(meta.out_indices[b])] = oracle.sdpa_row(q_source[int(meta.q_indices[b])].cpu(), kk, vv)
    return out


@pytest.mark.parametrize("bucket_tokens,single,splits", [(0, False, 4), (4096, False, 8),
                                                         (0, True, 20), (0, False, 1)])
def test_multi_bucket_step_matches_oracle(ext, gpu, bucket_tokens, single, splits):
    w = wl.config_c4()
    q_pool = wl.make_q_pool(w, gpu)
    k, v = wl.make_kv_pool(w, gpu)
    for i in (5, 30):
        step = serving.compile_bucket_step(w, i, gpu, splits, bucket_tokens=bucket_tokens,
                                           single_bucket=single)
        if not single:
            assert len(step.buckets) >= 2
        ws = serving.bucket_workspace(w, [step], gpu)
        out = serving.run_bucket_step(ext, w, step, i, q_pool, k, v, ws)
        torch.cuda.synchronize()
        eng_meta = serving.Engine.gate_meta(_Holder(step), 0)
        assert_parity(out, _oracle(w, eng_meta, q_pool[i], k, v))


class _Holder:
    """Engine.gate_meta reads .meta[i]; this holds one bucket step."""
    def __init__(self, step):
        self.meta = [("bucket", step)]


@pytest.mark.parametrize("name", ["c4", "c5_g8"])
def test_adaptive_engine_matches_oracle(ext, gpu, name):
    w = wl.CONFIGS[name]()
    eng = serving.Engine("adaptive", w, gpu)
    routes = {r for r, _ in eng.routes}
    assert routes <= {"persistentkv_bucket", "persistentkv_workqueue"}
    q_pool = wl.make_q_pool(w, gpu)
    k, v = wl.make_kv_pool(w, gpu)
    for i in (0, len(w.steps) // 2, len(w.steps) - 1):
        out = eng.run(ext, i, q_pool, k, v)
        torch.cuda.synchronize()
        assert_parity(out, _oracle(w, eng.gate_meta(i), q_pool[i], k, v))
        gate = serving.gate_step(out, eng.gate_meta(i), q_pool[i], k, v, w.page_size)
        assert gate["pass"], gate


def test_harness_run_reports_every_engine(ext, gpu):
    """One repeat of C3 at 32k through the three engines: the gate passes, timing and
    profiles are filled in, and the bucket engine launches one bucket per step."""
    rep = serving.run_workload(ext, "c3_32k", ["bucket", "workqueue", "adaptive"], 1, 2, 2, gpu,
                               wl.DEFAULT_SEED)
    assert set(rep["engines"]) == {"bucket", "workqueue", "adaptive"}
    for e in rep["engines"].values():
        assert e["gate"]["pass"]
        s = e["stats"]
        assert s["steps"] == rep["trace_steps"] and s["event_mean_ms"] > 0
        assert s["event_p50_ms"] <= s["event_p95_ms"] <= s["event_p99_ms"]
    assert rep["engines"]["bucket"]["profile"]["launches_per_step"] == 2.0
    assert "persistentkv_workqueue" in rep["engines"]["workqueue"]["profile"]["route_counts"]


def test_harness_fp8_engines_match_oracle(ext, gpu):
    """fp8 (e4m3) pools through the three engines: the bucket engine's
    paged_attention_indexed_fp8 launches, the work queue's paged_attention_workqueue_fp8 and
    the adaptive engine's routed steps each match the repack + fp32 SDPA oracle on the
    dequantised pages; a harness run passes its gate with every engine."""
    w = wl.config_c4()
    w.kv_fp8 = True
    q_pool = wl.make_q_pool(w, gpu)
    k, v = wl.make_kv_pool(w, gpu)
    assert k.dtype == torch.float8_e4m3fn
    kd, vd = serving.dequantize_pool(k, w.k_scale), serving.dequantize_pool(v, w.v_scale)
    for name in ("bucket", "workqueue", "adaptive"):
        eng = serving.Engine(name, w, gpu)
        for i in (3, len(w.steps) - 1):
            out = eng.run(ext, i, q_pool, k, v)
            torch.cuda.synchronize()
            assert_parity(out, _oracle(w, eng.gate_meta(i), q_pool[i], kd, vd))
    rep = serving.run_workload(ext, "c4", ["bucket", "workqueue", "adaptive"], 1, 1, 2, gpu,
                               wl.DEFAULT_SEED, kv_fp8=True)
    assert "fp8" in rep["dtype"]
    assert all(e["gate"]["pass"] for e in rep["engines"].values())


@pytest.mark.parametrize("engine", ["workqueue", "bucket", "adaptive"])
def test_reference_review_trace_step_matches_oracle(ext, gpu, engine):
    """The reference's seed-20260623 bimodal B8 review trace (scripts/run_review_ablations.sh:
    --trace bimodal --requests 24 --max-active 8 --steps 48 --hole-fraction 0.0, work-queue
    splits 20, bucket splits 32): its middle step through each engine, against the oracle."""
    w = wl.config_trace("bimodal", 24, 8, 48, 20260623, 0.0, 16, 8, 32, 20)
    assert w.physical_pages == 24285  # results/review_ablations/seed_20260623_bimodal_b8.txt:16
    eng = serving.Engine(engine, w, gpu, splits={"workqueue": 20, "bucket": 32}.get(engine))
    q_pool = wl.make_q_pool(w, gpu)
    k, v = wl.make_kv_pool(w, gpu)
    i = len(w.steps) // 2
    out = eng.run(ext, i, q_pool, k, v)
    torch.cuda.synchronize()
    print(f"engine={engine} step={i} lengths={w.steps[i].lengths}", flush=True)
    assert_parity(out, _oracle(w, eng.gate_meta(i), q_pool[i], k, v))


def test_trace_step_in_a_hip_graph_matches_eager(ext, gpu):
    """--graph: a captured step replayed (several times, with eager work between) gives the
    eager step's output bit for bit."""
    w = wl.config_trace("bucketed", 16, 1, 8, 20260623, 0.0, 16, 8, 32, 32)
    eng = serving.Engine("bucket", w, gpu, splits=32)
    q_pool = wl.make_q_pool(w, gpu)
    k, v = wl.make_kv_pool(w, gpu)
    eager = eng.run(ext, 3, q_pool, k, v).clone()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        eng.run(ext, 3, q_pool, k, v)
    for _ in range(3):
        eng.output(3).fill_(float("nan"))
        eng.run(ext, 5, q_pool, k, v)  # eager work on the same workspace between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(eng.output(3), eager)
