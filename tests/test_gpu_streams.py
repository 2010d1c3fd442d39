"""The direct op's internal split uses one scratch buffer per stream: ops on two streams
running at once must not see each other's partial states, and a launch captured into a
graph on a stream that has no buffer yet must fall back to the single-launch kernel and
replay correctly.  Gate: max-abs 2e-3, mean-abs 3e-4 against the fp32 oracle."""
import pytest
import torch

from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16 = torch.float16


def _direct(ext, case, gpu, out):
    q, k, v, bt = (x.to(gpu) for x in (case.q, case.k_pages, case.v_pages, case.block_table))
    empty = torch.empty(0, dtype=torch.float32, device=gpu)
    ctx = int(case.seq_lens[0])
    return lambda: ext.paged_attention(q, k, v, bt, out, empty, ctx, 16, 1)


def test_direct_split_on_two_streams_at_once(ext, gpu):
    cases = [make_case([2048], 32, 8, 16, F16, seed=s) for s in (31, 32)]
    outs = [torch.full((1, 32, 128), float("nan"), dtype=F16, device=gpu) for _ in cases]
    calls = [_direct(ext, c, gpu, o) for c, o in zip(cases, outs)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    for _ in range(20):  # interleave launches so the two streams' kernels overlap
        for st, call in zip(streams, calls):
            with torch.cuda.stream(st):
                call()
    torch.cuda.synchronize()
    for c, o in zip(cases, outs):
        ref = oracle.paged_decode(c.q, c.k_pages, c.v_pages, c.block_table, c.seq_lens)
        assert_parity(o, ref)


def test_direct_launch_captured_on_a_fresh_stream(ext, gpu):
    case = make_case([3000], 32, 8, 16, F16, seed=41)
    out = torch.zeros(1, 32, 128, dtype=F16, device=gpu)
    call = _direct(ext, case, gpu, out)
    side = torch.cuda.Stream()  # no eager launch on it: no scratch at capture time
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.synchronize()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    first = None
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(out, ref)
        first = out.clone() if first is None else first
        assert torch.equal(out, first)
    call()  # eager, on the current stream: the split path
    torch.cuda.synchronize()
    assert_parity(out, ref)
