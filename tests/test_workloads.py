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


def test_reference_review_traces_match_its_logs():
    """The two review traces the reference published step times for, rebuilt with its
    options: pool sizes as its logs print them, useful KV MiB per step as its profile
    table (results/review_ablations/seed_20260623_bimodal_b8.txt:16, :35;
    seed_20260623_bucketed_b1.txt:16, :35)."""
    w = wl.config_trace("bimodal", 24, 8, 48, 20260623, 0.0, 16, 8, 32, 20)
    assert w.physical_pages == 24285 and len(w.steps) == 48
    assert round(sum(w.kv_bytes(i) for i in range(48)) / 48 / 2 ** 20, 1) == 550.5
    w = wl.config_trace("bucketed", 16, 1, 64, 20260623, 0.0, 16, 8, 32, 32)
    assert w.physical_pages == 30793 and len(w.steps) == 64
    assert round(sum(w.kv_bytes(i) for i in range(64)) / 64 / 2 ** 20, 1) == 32.1
    assert all(len(s.active_ids) == 1 for s in w.steps)


def test_trace_file_loader(tmp_path):
    """load_trace_specs (benchmark_serving_trace.py:198-229): CSV and JSON, the field
    aliases, arrivals defaulting to the row index, prompts rounded up to pages, the
    request limit, and the error for a row without integer lengths."""
    csv_path = tmp_path / "t.csv"
    csv_path.write_text("prompt_len,decode_len,arrival\n100,5,0\n4096,7,2\n")
    assert wl.load_trace_specs(csv_path, 10) == [(0, 112, 5), (2, 4096, 7)]
    json_path = tmp_path / "t.json"
    json_path.write_text('[{"prompt": 17, "decode": 3}, {"prompt": 32, "decode": 4, "arrival_step": 9}]')
    assert wl.load_trace_specs(json_path, 10) == [(0, 32, 3), (9, 32, 4)]
    assert wl.load_trace_specs(json_path, 1) == [(0, 32, 3)]
    bad = tmp_path / "bad.csv"
    bad.write_text("prompt_len,decode_len\nx,5\n")
    with pytest.raises(ValueError, match="integer"):
        wl.load_trace_specs(bad, 10)
    w = wl.config_trace(trace_file=str(json_path), requests=10, max_active=1, steps=20,
                        hole_fraction=0.0)
    assert [r.arrival for r in w.requests] == [0, 9]
    assert w.steps[0].lengths == (32,) and w.steps[-1].active_ids == (1,)
