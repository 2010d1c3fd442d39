"""Pins the scheduling oracle (oracle/workqueue.py) on the CPU.

* Split policies and the cost-model router against vectors the reference's own functions
  produced (tests/golden/policy_vectors.json, written by make_policy_vectors.py).
* The compact work-queue builder against a hand-worked example and the builder's
  invariants (benchmark_serving_trace.py:668-729).
"""
import json
import os
import random

import pytest

from oracle import workqueue as wq

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "policy_vectors.json")


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as fh:
        return json.load(fh)


def test_row_splits_match_reference(golden):
    for hkv, length, active, req, auto, expected in golden["row_splits"]:
        assert wq.choose_workqueue_row_splits(length, active, req, bool(auto), hkv) == expected


def test_choose_splits_match_reference(golden):
    for hkv, lens, single, expected in golden["choose_splits"]:
        assert wq.choose_splits(lens, 16, True, bool(single), hkv) == expected


def test_model_splits_match_reference(golden):
    for hkv, lens, bucket, queue in golden["model_splits"]:
        assert wq.model_bucket_splits(lens, hkv) == bucket
        assert wq.model_workqueue_splits(lens, hkv) == queue


def test_cost_model_and_router_match_reference(golden):
    for hkv, lens, est, choice in golden["routes"]:
        cost = dict(wq.REFERENCE_COST, hkv=hkv)
        for route, pairs in est.items():
            for splits, ms in pairs:
                assert wq.estimate_route_ms(lens, route, splits, cost) == ms
        route, splits, ms = wq.choose_adaptive_route(lens, cost)
        assert [route, splits, ms] == choice


def test_builder_hand_worked_example():
    """lengths 64 / 100, 3 splits, 2 KV heads, page 16 — worked by hand:
    bucket 100 -> 7 table columns; row 0 has 2 tiles -> split ranges [0,0) [0,1) [1,2);
    row 1 has 4 tiles -> [0,1) [1,2) [2,4)."""
    got = wq.build_workqueue([64, 100], [5, 9], [[10, 11, 12, 13, 14], list(range(20, 28))], 16, 3,
                             False, hkv=2)
    assert got["block_table"] == [[10, 11, 12, 13, 14, 14, 14], [20, 21, 22, 23, 24, 25, 26]]
    assert got["work_items"] == [
        [0, 0, 1, 0, 1], [0, 1, 1, 0, 1], [0, 0, 2, 1, 2], [0, 1, 2, 1, 2],
        [1, 0, 0, 0, 1], [1, 1, 0, 0, 1], [1, 0, 1, 1, 2], [1, 1, 1, 1, 2],
        [1, 0, 2, 2, 4], [1, 1, 2, 2, 4]]
    assert got["split_offsets"] == [0, 3, 6]
    assert got["total_partial_slots"] == 6
    assert got["q_indices"] == [5, 9] and got["out_indices"] == [0, 1]
    assert got["seq_lens"] == [64, 100] and got["bucket_length"] == 100 and got["splits"] == 3


def check_builder_invariants(meta, lengths, hkv, page_lists, page_size):
    t = meta["work_items"]
    offs = meta["split_offsets"]
    assert offs[0] == 0 and len(offs) == len(lengths) + 1
    cols = -(-max(lengths) // page_size)
    for r, length in enumerate(lengths):
        items = [w for w in t if w[0] == r]
        total = (length + 31) // 32
        s = offs[r + 1] - offs[r]
        # ranges of the kvh-0 items tile [0, total) in split order
        ranges = [(w[3], w[4]) for w in items if w[1] == 0]
        assert [w[2] for w in items if w[1] == 0] == sorted(w[2] for w in items if w[1] == 0)
        if total:
            assert ranges[0][0] == 0 and ranges[-1][1] == total
        assert all(a[1] == b[0] for a, b in zip(ranges, ranges[1:]))
        assert len(ranges) == min(s, total)
        # each split appears once per KV head, KV heads innermost
        for i in range(0, len(items), hkv):
            assert [w[1] for w in items[i:i + hkv]] == list(range(hkv))
        row = meta["block_table"][r]
        assert len(row) == cols
        n = len(page_lists[r])
        assert row[:min(n, cols)] == list(page_lists[r][:cols])
        assert all(p == page_lists[r][-1] for p in row[n:])
    assert [w[0] for w in t] == sorted(w[0] for w in t)


def test_builder_invariants_random():
    rng = random.Random(7)
    for _ in range(300):
        n = rng.randint(1, 9)
        hkv = rng.choice([1, 2, 8])
        ps = rng.choice([8, 16, 32])
        lengths = [rng.randint(1, 3000) for _ in range(n)]
        page_lists = [list(range(1000 * r, 1000 * r + rng.randint(1, 200))) for r in range(n)]
        auto = rng.random() < 0.5
        meta = wq.build_workqueue(lengths, list(range(n)), page_lists, ps, rng.randint(1, 40), auto, hkv)
        check_builder_invariants(meta, lengths, hkv, page_lists, ps)


def test_round_bucket_length_matches_reference(golden):
    for page, length, bucket_tokens, pages, expected in golden["round_bucket"]:
        assert wq.round_bucket_length(length, bucket_tokens, pages, page) == expected


def test_round_bucket_length_hand_worked():
    """Worked by hand (page 16): 1000 tokens in 512-token buckets -> 1024; capped by the
    row's 40 allocated pages -> 640; bucket 100 -> 1000 rounds to 1000, then to the page
    multiple 1008; 7 tokens with 1-token buckets -> one page, 16; no bucketing -> 1000."""
    assert wq.round_bucket_length(1000, 512, 1000) == 1024
    assert wq.round_bucket_length(1000, 512, 40) == 640
    assert wq.round_bucket_length(1000, 100, 1000) == 1008
    assert wq.round_bucket_length(7, 1, 10) == 16
    assert wq.round_bucket_length(1000, 0, 1) == 1000


def test_planted_bucket_rounding_mistake_fails(golden):
    """A restatement that forgets the page rounding after the bucket rounding disagrees
    with the reference's vectors."""
    def wrong(length, bucket_tokens, pages, page):
        if bucket_tokens <= 0:
            return length
        return min(((length + bucket_tokens - 1) // bucket_tokens) * bucket_tokens, pages * page)
    assert any(wrong(length, b, pages, page) != expected
               for page, length, b, pages, expected in golden["round_bucket"])


def test_use_single_bucket_matches_reference(golden):
    for lens, single, adaptive, expected in golden["single_bucket"]:
        assert int(wq.use_single_bucket(lens, bool(single), bool(adaptive))) == expected


def test_bucket_builder_hand_worked_example():
    """Rows with lengths 300, 1000, 310, 1000 (page 16, 2 KV heads, 4 splits requested),
    exact buckets: 300 -> [row 0], 1000 -> [rows 1, 3], 310 -> [row 2], in that (first
    appearance) order; tables of ceil(300/16) = 19, 63 and 20 columns."""
    pages = [list(range(100, 119)), list(range(200, 263)), list(range(300, 320)),
             list(range(400, 463))]
    got = wq.build_buckets([300, 1000, 310, 1000], [7, 8, 9, 10], pages, 16, 4, False, hkv=2)
    assert [b["bucket_length"] for b in got] == [300, 1000, 310]
    assert [b["out_indices"] for b in got] == [[0], [1, 3], [2]]
    assert [b["q_indices"] for b in got] == [[7], [8, 10], [9]]
    assert [b["seq_lens"] for b in got] == [[300], [1000, 1000], [310]]
    assert [len(b["block_table"][0]) for b in got] == [19, 63, 20]
    assert got[1]["block_table"][1] == list(range(400, 463))
    assert all(b["splits"] == 4 for b in got)
    # 512-token buckets: 300, 310 and 1000 round up to 512 and 1024, then are capped at
    # each row's allocated pages (19, 20, 63 x 16 tokens), so the rows stay apart.
    got = wq.build_buckets([300, 1000, 310, 1000], [7, 8, 9, 10], pages, 16, 4, False,
                           bucket_tokens=512, hkv=2)
    assert [b["bucket_length"] for b in got] == [304, 1008, 320]
    # A single ragged bucket of max length; rows padded with their last page.
    got = wq.build_buckets([300, 1000, 310, 1000], [7, 8, 9, 10], pages, 16, 4, False,
                           single_bucket=True, hkv=2)
    assert len(got) == 1 and got[0]["bucket_length"] == 1000
    assert got[0]["block_table"][0] == list(range(100, 119)) + [118] * (63 - 19)


def check_bucket_invariants(buckets, lengths, request_ids, page_lists, page_size):
    seen = sorted(o for b in buckets for o in b["out_indices"])
    assert seen == list(range(len(lengths)))
    firsts = [b["out_indices"][0] for b in buckets]
    assert firsts == sorted(firsts)  # buckets in order of first appearance
    for b in buckets:
        cols = -(-b["bucket_length"] // page_size)
        assert b["out_indices"] == sorted(b["out_indices"])
        for row, o, n, q in zip(b["block_table"], b["out_indices"], b["seq_lens"], b["q_indices"]):
            assert n == lengths[o] and q == request_ids[o] and len(row) == cols
            p = page_lists[o]
            assert list(row[:len(p)]) == list(p[:cols]) and all(x == p[-1] for x in row[len(p):])


def test_bucket_builder_invariants_random():
    rng = random.Random(11)
    for _ in range(300):
        n = rng.randint(1, 9)
        ps = rng.choice([8, 16, 32])
        lengths = [rng.choice([rng.randint(1, 3000), 1024, 2048]) for _ in range(n)]
        page_lists = [list(range(1000 * r, 1000 * r + -(-lengths[r] // ps) + rng.randint(0, 5)))
                      for r in range(n)]
        b = rng.choice([0, 0, 256, 1000])
        got = wq.build_buckets(lengths, list(range(50, 50 + n)), page_lists, ps,
                               rng.randint(1, 40), rng.random() < 0.5, bucket_tokens=b,
                               single_bucket=rng.random() < 0.2, adaptive_route=rng.random() < 0.5,
                               hkv=rng.choice([1, 8]))
        check_bucket_invariants(got, lengths, list(range(50, 50 + n)), page_lists, ps)
