"""The C++ host scheduling in libpkv.so against the reference (golden vectors) and the
Python restatement, bit for bit; plus invariants of the MI355X split planner."""
import json
import os

import numpy as np
import pytest
from hypothesis import given, settings
from hypothesis import strategies as st

import pkv_native as nat
from oracle import workqueue as wq
from test_oracle_workqueue import GOLDEN, check_builder_invariants


@pytest.fixture(scope="module")
def golden():
    with open(GOLDEN) as fh:
        return json.load(fh)


def test_row_splits_match_reference(golden):
    for hkv, length, active, req, auto, expected in golden["row_splits"]:
        assert nat.choose_workqueue_row_splits(length, active, req, auto, hkv) == expected


def test_choose_and_model_splits_match_reference(golden):
    for hkv, lens, single, expected in golden["choose_splits"]:
        assert nat.choose_splits(lens, 16, True, single, hkv) == expected
    for hkv, lens, bucket, queue in golden["model_splits"]:
        assert nat.model_bucket_splits(lens, hkv) == bucket
        assert nat.model_workqueue_splits(lens, hkv) == queue


def test_cost_model_and_router_match_reference(golden):
    for hkv, lens, est, choice in golden["routes"]:
        m = nat.cost_model(nat.POLICY_REFERENCE, num_kv_heads=hkv)
        for route, pairs in est.items():
            for splits, ms in pairs:
                assert nat.estimate_route_ms(lens, route, splits, m) == ms
        assert list(nat.choose_adaptive_route(lens, m)) == choice


@settings(max_examples=300, deadline=None)
@given(st.lists(st.integers(1, 40000), min_size=1, max_size=10), st.integers(1, 48),
       st.booleans(), st.sampled_from([1, 2, 4, 8, 32]), st.sampled_from([8, 16, 32, 64]),
       st.integers(0, 1 << 30))
def test_builder_matches_python_restatement(lengths, requested, auto, hkv, ps, seed):
    rng = np.random.default_rng(seed)
    n = len(lengths)
    page_lists = [list(rng.integers(0, 1 << 20, size=int(rng.integers(1, 3000 // ps + 2)))) for _ in range(n)]
    ids = [int(x) for x in rng.permutation(n + 3)[:n]]
    py = wq.build_workqueue(lengths, ids, page_lists, ps, requested, auto, hkv)
    cc = nat.build_workqueue(lengths, ids, page_lists, ps, requested, auto, hkv)
    assert cc["block_table"].tolist() == py["block_table"]
    assert cc["work_items"].tolist() == py["work_items"]
    assert cc["split_offsets"].tolist() == py["split_offsets"]
    assert cc["seq_lens"].tolist() == py["seq_lens"]
    assert cc["q_indices"].tolist() == py["q_indices"]
    assert cc["out_indices"].tolist() == py["out_indices"]
    assert cc["total_partial_slots"] == py["total_partial_slots"]
    assert cc["bucket_length"] == py["bucket_length"] and cc["splits"] == py["splits"]


def test_mi355x_planner_invariants():
    rng = np.random.default_rng(3)
    for _ in range(200):
        n = int(rng.integers(1, 65))
        lengths = [int(x) for x in rng.integers(1, 70000, size=n)]
        hkv = int(rng.choice([1, 4, 8, 32]))
        group = int(rng.choice([1, 4, 8, 16, 32]))
        pages = [list(range(-(-x // 16) + 1)) for x in lengths]
        meta = nat.build_workqueue(lengths, list(range(n)), pages, 16, 1, True, hkv, nat.POLICY_MI355X,
                                   hq=hkv * group)
        m = {k: (v.tolist() if hasattr(v, "tolist") else v) for k, v in meta.items()}
        check_builder_invariants(m, lengths, hkv, pages, 16)
        row_splits = np.diff(meta["split_offsets"])
        tiles = np.array([(x + 31) // 32 for x in lengths])
        assert np.all(row_splits >= 1) and np.all(row_splits <= np.maximum(tiles, 1))
        # no empty splits: every slot has work
        assert len(meta["work_items"]) == int(row_splits.sum()) * hkv
        # G > 16 (the two-head-block kernel): every item starts in the first round on 256
        # CUs, unless the rows alone (one split each) are more than that
        if group > 16:
            assert len(meta["work_items"]) <= max(256, n * hkv)


def test_mi355x_planner_wide_group_takes_the_smallest_item_that_fits():
    """G > 16: the split of every row is ceil(tiles / M) (at most 128) for the smallest item
    size M (at least 8 tiles and the step's mean share of 256 CUs) at which the step has at
    most 256 items, found here by brute force; the launch lasts as long as its largest
    item."""
    rng = np.random.default_rng(11)
    for _ in range(60):
        n = int(rng.integers(1, 70))
        lengths = [int(x) for x in rng.integers(1, 66000, size=n)]
        hkv = int(rng.choice([1, 2]))
        tiles = [max(1, (x + 31) // 32) for x in lengths]
        items_at = lambda m: sum(max(1, min(-(-t // m), 128)) for t in tiles) * hkv
        m = max(8, -(-sum(tiles) * hkv // 256))
        while items_at(m) > 256 and m < max(tiles):
            m += 1
        pages = [list(range(-(-x // 16) + 1)) for x in lengths]
        meta = nat.build_workqueue(lengths, list(range(n)), pages, 16, 1, True, hkv,
                                   nat.POLICY_MI355X, hq=32 * hkv)
        expected = [max(1, min(-(-t // m), 128)) for t in tiles]
        assert np.diff(meta["split_offsets"]).tolist() == expected


def test_c4_step_uses_twenty_splits():
    lengths = [20000, 300, 700, 256, 1024, 512, 600, 31000]
    meta = nat.build_workqueue(lengths, list(range(8)), [list(range(-(-x // 16))) for x in lengths],
                               16, 20, False, 8)
    assert meta["total_partial_slots"] == 160
    assert np.all(np.diff(meta["split_offsets"]) == 20)


def test_bucket_functions_match_reference(golden):
    for page, length, bucket_tokens, pages, expected in golden["round_bucket"]:
        assert nat.round_bucket_length(length, bucket_tokens, pages, page) == expected
    for lens, single, adaptive, expected in golden["single_bucket"]:
        assert int(nat.use_single_bucket(lens, single, adaptive)) == expected


@settings(max_examples=300, deadline=None)
@given(st.lists(st.integers(1, 40000), min_size=1, max_size=10), st.integers(1, 48),
       st.booleans(), st.sampled_from([0, 0, 256, 1000, 4096]), st.booleans(), st.booleans(),
       st.sampled_from([1, 2, 8, 32]), st.sampled_from([8, 16, 32, 64]), st.integers(0, 1 << 30))
def test_bucket_builder_matches_python_restatement(lengths, requested, auto, bucket_tokens, single,
                                                   adaptive, hkv, ps, seed):
    rng = np.random.default_rng(seed)
    n = len(lengths)
    # repeated lengths so that rows share buckets
    lengths = [lengths[int(rng.integers(0, n))] if rng.random() < 0.4 else x for x in lengths]
    page_lists = [list(rng.integers(0, 1 << 20, size=int(rng.integers(1, 3000 // ps + 2)))) for _ in range(n)]
    ids = [int(x) for x in rng.permutation(n + 3)[:n]]
    py = wq.build_buckets(lengths, ids, page_lists, ps, requested, auto, bucket_tokens, single,
                          adaptive, hkv)
    cc = nat.build_buckets(lengths, ids, page_lists, ps, requested, auto, bucket_tokens, single,
                           adaptive, hkv)
    assert len(cc) == len(py)
    for c, p in zip(cc, py):
        assert c["bucket_length"] == p["bucket_length"] and c["splits"] == p["splits"]
        assert c["block_table"].tolist() == p["block_table"]
        assert c["seq_lens"].tolist() == p["seq_lens"]
        assert c["q_indices"].tolist() == p["q_indices"]
        assert c["out_indices"].tolist() == p["out_indices"]


def test_mi355x_router_never_leaves_the_engine(golden):
    """The MI355X policy routes every step to one of the engine's own routes (split grid or
    work queue), for every G, length and active count; the reference policy keeps its
    FlashInfer fallback (pinned by test_cost_model_and_router_match_reference)."""
    lens_grid = [1, 31, 32, 256, 2048, 8192, 16383, 16384, 32768, 65536, 131072]
    cases = [[x] * n for x in lens_grid for n in (1, 2, 3, 4, 7, 8, 9, 16, 64)]
    cases += [lens for _, lens, _, _ in golden["routes"]]
    cases += [lens for _, lens, _, _ in golden["model_splits"]]
    cases += [[2048], [20000, 30000, 300], [20000] * 4]
    routes = set()
    for hq, hkv in ((32, 8), (32, 1), (32, 4), (32, 32), (48, 2), (27, 1)):
        m = nat.cost_model(nat.POLICY_MI355X, num_q_heads=hq, num_kv_heads=hkv)
        for lens in cases:
            route, splits, ms = nat.choose_adaptive_route(lens, m)
            assert route in ("persistentkv_bucket", "persistentkv_workqueue"), (hq, hkv, lens)
            assert splits >= 1 and ms > 0
            routes.add(route)
    assert routes == {"persistentkv_bucket", "persistentkv_workqueue"}


def test_mi355x_router_choices():
    """The MI355X cost model's choices on the configs' shapes: equal rows run the split
    grid with one unit per CU (B1 Hkv 8: 32 splits; the direct launch's own split count);
    mixed lengths run the balanced work queue."""
    m = nat.cost_model(nat.POLICY_MI355X, num_q_heads=32, num_kv_heads=8)
    for lens in ([32768], [16384], [2048], [8192]):
        route, splits, _ = nat.choose_adaptive_route(lens, m)
        assert (route, splits) == ("persistentkv_bucket", 32), lens
    route, _, _ = nat.choose_adaptive_route([20000, 300, 700, 256, 1024, 512, 600, 31000], m)
    assert route == "persistentkv_workqueue"
    mha = nat.cost_model(nat.POLICY_MI355X, num_q_heads=32, num_kv_heads=32)
    assert nat.choose_adaptive_route([4096] * 8, mha)[:2] == ("persistentkv_bucket", 1)
    for hkv in (1, 4):
        zipf = [128 + (65536 - 128) // (i + 1) ** 2 for i in range(64)]
        m = nat.cost_model(nat.POLICY_MI355X, num_q_heads=32, num_kv_heads=hkv)
        assert nat.choose_adaptive_route(zipf, m)[0] == "persistentkv_workqueue"


def test_mi355x_grid_split_rule():
    """pkv_choose_splits (MI355X): one unit per CU for rows of one length; for mixed
    lengths, units of the longest row at most a quarter of a CU's tile share; at least
    two tiles per unit of the longest row."""
    P = nat.POLICY_MI355X
    assert nat.choose_splits([32768], 1, True, False, 8, P) == 32        # 8 x 32 = 256 units
    assert nat.choose_splits([4096] * 8, 1, True, False, 8, P) == 4      # 8 x 8 x 4 = 256
    assert nat.choose_splits([4096] * 8, 1, True, False, 32, P) == 1     # 256 rows x heads
    assert nat.choose_splits([100], 1, True, False, 8, P) == 2           # 4 tiles: 2 per unit
    lens = [1024 + 900 * i for i in range(8)]                            # C2-like, MHA
    tiles = [(x + 31) // 32 for x in lens]
    s = nat.choose_splits(lens, 1, True, False, 32, P)
    assert -(-max(tiles) // s) <= 32 * sum(tiles) / 256 / 4 + 1
    assert s == -(-4 * max(tiles) * 256 // (32 * sum(tiles)))
