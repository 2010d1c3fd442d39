"""The direct op (num_splits == 1) splits itself internally into the caller's workspace
when it is large enough, and allocates nothing: every launch with its own workspace is
independent of other streams and of the launch history, and a captured launch replays
the eager result.  Gate: max-abs 2e-3, mean-abs 3e-4 against the fp32 oracle."""
import pytest
import torch

from oracle import attention as oracle
from paged_cases import assert_parity, make_case

pytestmark = pytest.mark.gpu
F16 = torch.float16


def _direct(ext, case, gpu, out, ws):
    q, k, v, bt = (x.to(gpu) for x in (case.q, case.k_pages, case.v_pages, case.block_table))
    ctx = int(case.seq_lens[0])
    return lambda: ext.paged_attention(q, k, v, bt, out, ws, ctx, 16, 1)


def _ws(floats, gpu):
    return torch.empty(floats, dtype=torch.float32, device=gpu)


def test_direct_split_uses_the_callers_workspace(ext, gpu):
    case = make_case([2048], 32, 8, 16, F16, seed=30)
    full = ext.direct_workspace_floats(1, 32, 8, 2048)
    assert full == 32 * 32 * 130  # 8 (row, kv head) pairs -> 32 splits of 2 tiles
    assert ext.direct_workspace_floats(1, 32, 8, 32) == 0  # one tile: nothing to split
    assert ext.direct_workspace_floats(16, 32, 8, 4096) == 0  # 128 units: not split
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    outs = []
    for floats in (0, full // 4, full, 4 * full):  # single launch, 8, 32 and 32 splits
        out = torch.full((1, 32, 128), float("nan"), dtype=F16, device=gpu)
        _direct(ext, case, gpu, out, _ws(floats, gpu))()
        torch.cuda.synchronize()
        assert_parity(out, ref)
        outs.append(out.float())
    for o in outs[1:]:
        assert (o - outs[0]).abs().max().item() < 1e-3
    assert torch.equal(outs[2], outs[3])


def test_direct_split_on_two_streams_at_once(ext, gpu):
    cases = [make_case([2048], 32, 8, 16, F16, seed=s) for s in (31, 32)]
    outs = [torch.full((1, 32, 128), float("nan"), dtype=F16, device=gpu) for _ in cases]
    full = ext.direct_workspace_floats(1, 32, 8, 2048)
    calls = [_direct(ext, c, gpu, o, _ws(full, gpu)) for c, o in zip(cases, outs)]
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


@pytest.mark.parametrize("with_workspace", [False, True])
def test_direct_launch_captured_on_a_fresh_stream(ext, gpu, with_workspace):
    """Captured with no eager launch before it: the replay equals the eager launch bit for
    bit, with the internal split (workspace) or the single launch (empty workspace)."""
    case = make_case([3000], 32, 8, 16, F16, seed=41)
    out = torch.zeros(1, 32, 128, dtype=F16, device=gpu)
    floats = ext.direct_workspace_floats(1, 32, 8, 3000) if with_workspace else 0
    ws = _ws(floats, gpu)
    call = _direct(ext, case, gpu, out, ws)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call()
    torch.cuda.synchronize()
    call()  # eager, on the current stream
    torch.cuda.synchronize()
    eager = out.clone()
    ref = oracle.paged_decode(case.q, case.k_pages, case.v_pages, case.block_table, case.seq_lens)
    assert_parity(eager, ref)
    for _ in range(3):
        out.zero_()
        if floats:
            ws.fill_(7.0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
