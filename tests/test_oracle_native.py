"""Pins the C restatement of the oracle (oracle/pkv_oracle.c via oracle/native.py).

Checks, all on the CPU:
  * the reference's exact CPU attention (smoke_test.cu:35-74) against the fp64 brute force
    on each of the eight smoke-case inputs, and the committed expected outputs against it;
  * the smoke inputs against glibc's rand() stream drawn independently here: case c's
    first Q value sits at the offset that Q, K, V of all earlier cases consume;
  * split partial states against the fp64 partial states of oracle/attention.py (which are
    pinned there by split invariance), including the empty range's neutral state;
  * split + merge decode against the fp32 SDPA oracle for several split counts and
    page tables;
  * a planted mistake (partials in log2 units) failing the same comparison.
"""
import ctypes
import os

import numpy as np
import pytest
import torch

from oracle import attention as oracle
from oracle import native
from paged_cases import make_case

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "smoke_expected.npz")
NEG_FLT_MAX = float(-np.finfo(np.float32).max)


def _contiguous_fp64(q, k, v, b):
    """fp64 attention of batch row b of contiguous smoke inputs."""
    return oracle.attention_fp64(torch.from_numpy(q[b]), torch.from_numpy(k[b]),
                                 torch.from_numpy(v[b]))


@pytest.mark.parametrize("index", range(native.SMOKE_CASES))
def test_cpu_gqa_attention_matches_fp64(index):
    q, k, v = (x.astype(np.float16).astype(np.float32) for x in native.smoke_inputs(index))
    got = native.cpu_gqa_attention(q, k, v)
    golden = np.load(GOLDEN)[f"expected_{index}"]
    for b in range(q.shape[0]):
        exact = _contiguous_fp64(q, k, v, b)
        assert np.abs(got[b] - exact).max() < 2e-6
        assert np.abs(golden[b] - exact).max() < 2e-6


def test_smoke_inputs_follow_the_glibc_stream():
    libc = ctypes.CDLL("libc.so.6")
    libc.srand(42)
    cases = [native.smoke_case(i) for i in range(3)]
    draws = sum(b * hq * 128 + 2 * b * hkv * n * 128 for b, hq, hkv, n, _, _ in cases)
    stream = np.array([libc.rand() for _ in range(draws)], dtype=np.int64)
    values = stream.astype(np.float32) / np.float32(2147483647) * np.float32(2) - np.float32(1)
    offset = 0
    for index in range(3):
        b, hq, hkv, n, _, _ = native.smoke_case(index)
        q, k, v = native.smoke_inputs(index)
        qn, kvn = b * hq * 128, b * hkv * n * 128
        np.testing.assert_array_equal(q.ravel(), values[offset:offset + qn])
        np.testing.assert_array_equal(k.ravel()[:64], values[offset + qn:offset + qn + 64])
        np.testing.assert_array_equal(v.ravel()[-64:],
                                      values[offset + qn + 2 * kvn - 64:offset + qn + 2 * kvn])
        offset += qn + 2 * kvn


@pytest.mark.parametrize("length,ranges", [(300, [(0, 3), (3, 7), (7, 10), (10, 10)]),
                                           (33, [(0, 1), (1, 2)]), (64, [(0, 2)])])
def test_split_partial_matches_fp64_partials(length, ranges):
    case = make_case([length], 8, 2, 16, torch.float16, seed=length)
    kf, vf = case.k_pages.float().numpy(), case.v_pages.float().numpy()
    table = case.block_table[0].numpy()
    k, v = oracle.gather_row(case.k_pages, case.v_pages, case.block_table[0], length)
    m64, l64, acc64 = oracle.split_partials(case.q[0], k, v, ranges)
    for h in (0, 3, 5):
        for i, (tb, te) in enumerate(ranges):
            m, l, acc = native.split_partial(case.q[0, h].float().numpy(), kf, vf, table, 16,
                                             h // 4, length, tb, te)
            if te * 32 <= tb * 32 or tb * 32 >= length:
                assert (m, l) == (NEG_FLT_MAX, 0.0) and not acc.any()
                continue
            assert abs(m - m64[h, i]) < 1e-5
            assert abs(l - l64[h, i]) < 1e-5 * l64[h, i]
            assert np.abs(acc - acc64[h, i]).max() < 1e-4


def test_merge_identity_and_empty_merge():
    rng = np.random.default_rng(3)
    m = rng.normal(size=3).astype(np.float32)
    l = rng.uniform(1, 5, size=3).astype(np.float32)
    acc = rng.normal(size=(3, 128)).astype(np.float32)
    out = np.zeros(128, dtype=np.float32)
    native.lib().pkv_oracle_lse_merge(m, l, acc, 3, out)
    m4 = np.append(m, np.float32(NEG_FLT_MAX)).astype(np.float32)
    l4 = np.append(l, np.float32(0)).astype(np.float32)
    acc4 = np.vstack([acc, np.zeros((1, 128), np.float32)])
    out4 = np.zeros(128, dtype=np.float32)
    native.lib().pkv_oracle_lse_merge(m4, l4, acc4, 4, out4)
    np.testing.assert_array_equal(out, out4)
    np.testing.assert_allclose(out, oracle.lse_merge(m.astype(np.float64), l.astype(np.float64),
                                                     acc.astype(np.float64)), atol=1e-6)
    zero = np.ones(128, dtype=np.float32)
    native.lib().pkv_oracle_lse_merge(m4[3:], l4[3:], acc4[3:], 1, zero)
    assert not zero.any()


@pytest.mark.parametrize("table", ["random", "reversed", "canonical"])
@pytest.mark.parametrize("splits", [1, 3, 7])
def test_paged_decode_matches_sdpa_oracle(table, splits):
    length = 288 if table == "canonical" else 250
    case = make_case([length], 8, 2, 16, torch.float16, seed=splits, table=table)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                              case.seq_lens)[0].numpy()
    got = native.paged_decode_row(case.q[0].float().numpy(), case.k_pages.float().numpy(),
                                  case.v_pages.float().numpy(), case.block_table[0].numpy(), 16,
                                  length, splits)
    assert np.abs(got - ref).max() < 2e-6


def test_log2_partials_mistake_is_caught():
    """Partials kept in log2 units (a plausible slip when exp2 is used) break the merge."""
    length, ranges = 200, [(0, 3), (3, 7)]
    case = make_case([length], 4, 1, 16, torch.float16, seed=9)
    kf, vf = case.k_pages.float().numpy(), case.v_pages.float().numpy()
    table = case.block_table[0].numpy()
    parts = [native.split_partial(case.q[0, 0].float().numpy(), kf, vf, table, 16, 0, length,
                                  tb, te) for tb, te in ranges]
    m = np.array([p[0] for p in parts], np.float32)
    l = np.array([p[1] for p in parts], np.float32)
    acc = np.vstack([p[2] for p in parts]).astype(np.float32)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table,
                              case.seq_lens)[0, 0].numpy()
    out = np.zeros(128, np.float32)
    native.lib().pkv_oracle_lse_merge(m, l, acc, 2, out)
    assert np.abs(out - ref).max() < 2e-6
    bad = np.zeros(128, np.float32)
    native.lib().pkv_oracle_lse_merge((m * np.float32(1.4426950)).astype(np.float32), l, acc, 2, bad)
    assert np.abs(bad - ref).max() > 1e-4
