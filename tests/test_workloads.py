"""Trace mechanics of the serving harness (persistentkv-attention_amd/pkv_workloads.py)
against golden traces written by the reference's own make_lengths / build_requests /
build_steps (tests/benchmark_serving_trace.py:159-298; tests/golden/make_policy_vectors.py):
request lengths, pool size, every request's page list (count, first ids, CRC32 of all ids),
arrivals and every step's active set and lengths, bit-exact.  Also the configuration
builders' invariants (page lists disjoint, lengths within the reserved pages)."""
import json
import os
import struct
import zlib

import pytest

import pkv_workloads as wl

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "policy_vectors.json")
TRACES = json.load(open(GOLDEN))["traces"]


@pytest.mark.parametrize("t", TRACES, ids=lambda t: f"{t['trace']}-{t['seed']}-p{t['page_size']}")
def test_trace_matches_reference_vectors(t):
    lengths = wl.make_lengths(t["trace"], t["requests"], t["seed"], t["page_size"])
    assert [list(x) for x in lengths] == t["lengths"]
    reqs, physical = wl.build_requests(lengths, t["max_active"], t["seed"], t["hole_fraction"],
                                       t["page_size"])
    assert physical == t["physical_pages"]
    for req, (count, first, crc) in zip(reqs, t["pages"]):
        assert len(req.physical_pages) == count
        assert list(req.physical_pages[:4]) == first
        assert zlib.crc32(struct.pack(f"<{count}i", *req.physical_pages)) == crc
    assert [r.arrival for r in reqs] == t["arrivals"]
    steps = wl.build_steps(reqs, t["max_active"])
    assert [[s.step, list(s.active_ids), list(s.lengths)] for s in steps] == t["steps"]


@pytest.mark.parametrize("name", sorted(wl.CONFIGS))
def test_config_pages_are_disjoint_and_cover_every_step(name):
    w = wl.CONFIGS[name]()
    seen = set()
    for r in w.requests:
        assert not seen.intersection(r.physical_pages)
        seen.update(r.physical_pages)
    by_id = {r.request_id: r for r in w.requests}
    for st in w.steps:
        assert len(st.active_ids) <= len(w.requests)
        for rid, length in zip(st.active_ids, st.lengths):
            assert 0 < length <= len(by_id[rid].physical_pages) * w.page_size
