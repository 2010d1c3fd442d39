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
