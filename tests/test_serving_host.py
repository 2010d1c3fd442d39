"""Host-side pieces of the serving harness (pkv_serving) on the CPU.

* The correctness gate's torch fp32 reference equals the oracle's repack + SDPA on the
  same pages, and the gate fails an output with a planted error.
* The latency summary follows the reference's percentile rule
  (benchmark_serving_trace.py:1029-1036).
* Route profiles count launches and non-empty CTAs as the reference does (:516-616).
"""
from dataclasses import dataclass

import torch

import pkv_serving as serving
import pkv_workloads as wl
from oracle import attention as oracle
from paged_cases import make_case


@dataclass
class _Meta:
    block_table: torch.Tensor
    seq_lens: torch.Tensor
    q_indices: torch.Tensor
    out_indices: torch.Tensor
    output: torch.Tensor


def _case(dtype):
    case = make_case([300, 17, 1000, 64], 32, 8, 16, dtype, seed=5, q_rows=6)
    qi = torch.tensor([5, 0, 2, 3], dtype=torch.int32)
    oi = torch.tensor([1, 0, 3, 2], dtype=torch.int32)
    meta = _Meta(case.block_table, case.seq_lens, qi, oi, torch.empty(4, 32, 128, dtype=dtype))
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens,
                              qi, oi)
    return case, meta, ref


def test_gate_reference_equals_oracle():
    case, meta, ref = _case(torch.float16)
    got = serving.reference_step(meta, case.q, case.k_pages, case.v_pages, 16)
    assert (got - ref).abs().max().item() < 1e-5


def test_gate_passes_the_oracle_and_fails_a_planted_error():
    for dtype in (torch.float16, torch.bfloat16):
        case, meta, ref = _case(dtype)
        good = serving.gate_step(ref.to(dtype), meta, case.q, case.k_pages, case.v_pages, 16)
        assert good["pass"], good
        bad = ref.clone()
        bad[2, 7, 5] += 0.01  # one element off by 1e-2
        res = serving.gate_step(bad.to(dtype), meta, case.q, case.k_pages, case.v_pages, 16)
        assert not res["pass"] and res["max_abs"] > 5e-3


def test_latency_summary_percentiles():
    samples = [float(x) for x in range(1, 101)]  # 1 .. 100
    mean, p50, p95, p99 = serving.summarize(samples[::-1])
    assert (mean, p50, p95, p99) == (50.5, 50.0, 95.0, 99.0)
    assert serving.summarize([3.0]) == (3.0, 3.0, 3.0, 3.0)
    assert serving.summarize([]) == (0.0, 0.0, 0.0, 0.0)


def test_bucket_profile_counts():
    """Two buckets on Hkv 8: 3 splits over rows of 2 and 5 tiles (one split of the 2-tile
    row is empty), and 1 split (a direct launch, no merge)."""
    w = wl.config_c4()
    b1 = serving.Bucket(160, torch.zeros(2, 10, dtype=torch.int32),
                        torch.tensor([33, 160], dtype=torch.int32), torch.zeros(2, dtype=torch.int32),
                        torch.zeros(2, dtype=torch.int32), 3, 3)
    b2 = serving.Bucket(40, torch.zeros(1, 3, dtype=torch.int32), torch.tensor([40], dtype=torch.int32),
                        torch.zeros(1, dtype=torch.int32), torch.zeros(1, dtype=torch.int32), 1, 1)
    step = serving.BucketStep([b1, b2], torch.empty(3, 32, 128), 0)
    launches, nonempty, ctas, merge_mb, merges = serving.step_profile(w, "bucket", step)
    assert launches == 3 and merges == 1
    assert nonempty == (2 + 3 + 1) * 8 / ((2 * 3 + 1) * 8)
    assert ctas == (2 * 8 * 3 + 8) / 256
    assert merge_mb == 2 * 32 * 3 * 130 * 4 / 2 ** 20
