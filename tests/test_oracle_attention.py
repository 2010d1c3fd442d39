"""Pins the attention oracle (oracle/attention.py) on the CPU.

Checks: fp64 brute force, closed forms (equal keys give the mean of V; a dominant key
selects its V row), identity / reversed / canonical page tables, split invariance of the
partial states + LSE merge, the neutral state as merge identity, permutation invariance,
and that plausible mistakes (wrong GQA head mapping, missing softmax scale, a dropped
token) fail the same comparisons.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oracle
from paged_cases import make_case


def _row(case, b=0):
    n = int(case.seq_lens[b])
    return oracle.gather_row(case.k_pages, case.v_pages, case.block_table[b], n)


@pytest.mark.parametrize("hq,hkv,n,ps,dtype", [
    (4, 1, 257, 16, torch.float16), (8, 2, 33, 8, torch.float16), (32, 8, 300, 16, torch.float16),
    (32, 32, 64, 32, torch.bfloat16), (32, 1, 129, 5, torch.bfloat16), (12, 4, 1, 16, torch.float16)])
def test_sdpa_matches_fp64(hq, hkv, n, ps, dtype):
    case = make_case([n, n // 2 + 1], hq, hkv, ps, dtype, seed=n)
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    for b in range(2):
        k, v = _row(case, b)
        exact = oracle.attention_fp64(case.q[b], k, v)
        assert np.abs(ref[b].numpy() - exact).max() < 2e-5


def test_gather_identity_and_reversed_tables():
    cont = make_case([100, 77], 8, 2, 16, seed=1, table="contiguous", extra_pages=0)
    k0, v0 = _row(cont, 1)
    # contiguous pages: token t of row 1 is page (7 + t // 16), offset t % 16 (row 0 has 7 pages)
    pool_k = cont.k_pages
    for t in (0, 15, 16, 76):
        assert torch.equal(k0[:, t], pool_k[7 + t // 16, :, t % 16])
    rev = make_case([100], 8, 2, 16, seed=1, table="reversed", extra_pages=0)
    k1, _ = _row(rev)
    for t in (0, 31, 99):
        assert torch.equal(k1[:, t], rev.k_pages[6 - t // 16, :, t % 16])


def test_canonical_table_closed_form():
    for ctx in (8192, 32768, 65536):
        t = oracle.canonical_block_table(ctx)
        assert len(t) == ctx // 16 and len(set(t)) == len(t)
        assert all(0 <= p < 2 * (ctx // 16) for p in t)
        assert t[:3] == [17, 422, 827 % (2 * (ctx // 16))]


def test_uniform_keys_give_mean_of_values():
    case = make_case([200], 8, 2, 16, seed=2)
    case.k_pages[:] = case.k_pages[0:1, :, 0:1]   # every token has the same key per head
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    _, v = _row(case)
    for h in range(8):
        np.testing.assert_allclose(ref[0, h].numpy(), v[h // 4].float().mean(0).numpy(), atol=1e-5)


def test_dominant_key_selects_its_value():
    case = make_case([96], 4, 1, 16, seed=3, dtype=torch.float32)
    k, v = _row(case)
    target = 37
    page, off = case.page_lists[0][target // 16], target % 16
    case.k_pages[page, 0, off] = case.q[0, 0] * 100.0
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    np.testing.assert_allclose(ref[0, 0].numpy(), v[0, target].numpy(), atol=1e-4)


@pytest.mark.parametrize("n,splits", [(1, 1), (31, 4), (257, 4), (259, 3), (1000, 17), (64, 48)])
def test_split_partials_merge_to_unsplit(n, splits):
    case = make_case([n], 8, 2, 16, seed=n)
    k, v = _row(case)
    ranges = oracle.split_bounds(-(-n // 32), splits)
    m, l, acc = oracle.split_partials(case.q[0], k, v, ranges)
    merged = oracle.lse_merge(m, l, acc)
    np.testing.assert_allclose(merged, oracle.attention_fp64(case.q[0], k, v), atol=1e-12)
    # the neutral state (-FLT_MAX, 0, 0) is the merge identity
    m2 = np.concatenate([m, np.full((8, 1), float(oracle.NEG_FLT_MAX))], 1)
    l2 = np.concatenate([l, np.zeros((8, 1))], 1)
    acc2 = np.concatenate([acc, np.zeros((8, 1, 128))], 1)
    np.testing.assert_array_equal(oracle.lse_merge(m2, l2, acc2), merged)


def test_split_bounds_partition():
    for total in range(0, 70):
        for s in range(1, 50):
            r = oracle.split_bounds(total, s)
            assert r[0][0] == 0 and r[-1][1] == total
            assert all(a[1] == b[0] for a, b in zip(r, r[1:]))
            assert sum(1 for a, b in r if b > a) == min(s, total)


def test_token_permutation_invariance():
    case = make_case([150], 8, 2, 16, seed=4)
    k, v = _row(case)
    perm = torch.randperm(150, generator=torch.Generator().manual_seed(0))
    a = oracle.attention_fp64(case.q[0], k, v)
    b = oracle.attention_fp64(case.q[0], k[:, perm], v[:, perm])
    np.testing.assert_allclose(a, b, atol=1e-12)


def test_plausible_mistakes_are_caught():
    """Each mutation of the math must move the result far beyond the 2e-3 tolerance."""
    case = make_case([300], 32, 8, 16, seed=5, dtype=torch.float32)
    k, v = _row(case)
    good = oracle.attention_fp64(case.q[0], k, v)
    q = case.q[0].double().numpy()
    kk, vv = k.double().numpy(), v.double().numpy()

    def attend(kvh_of, scale=oracle.SCALE, drop_last=False):
        out = np.zeros((32, 128))
        for h in range(32):
            kh, vh = kk[kvh_of(h)], vv[kvh_of(h)]
            if drop_last:
                kh, vh = kh[:-1], vh[:-1]
            s = kh @ q[h] * scale
            p = np.exp(s - s.max())
            out[h] = p @ vh / p.sum()
        return out

    np.testing.assert_allclose(attend(lambda h: h // 4), good, atol=1e-12)
    assert np.abs(attend(lambda h: h % 8) - good).max() > 1e-2      # wrong GQA mapping
    assert np.abs(attend(lambda h: h // 4, scale=1.0) - good).max() > 1e-2  # missing scale
    assert np.abs(attend(lambda h: h // 4, drop_last=True) - good).max() > 1e-4  # dropped token
