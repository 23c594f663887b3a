"""Selection, forward and backward captured in one HIP graph (torch.cuda.CUDAGraph) and replayed.

The library records no memset, allocation or host synchronisation when max_seqlen is given
(workspaces come from torch's allocator, inside a capture from the graph's pool), so a caller
can capture a whole step.  Every replay -- with eager steps and synchronisations between the
replays -- must equal the eager results bit for bit.  Two steps on two streams at once must
equal the same steps run one after the other.
"""
from __future__ import annotations

import pytest
import torch

from dsalt_amd import ops
from dsalt_amd.workloads import WORKLOADS, generate

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name,seqlen", [("fwdbwd_bf16_h16_l32768", 4096), ("fwd_bf16_h16_l131072_block", 4096),
                                         ("fwdbwd_bf16_b4_h8_l8192", 2048)])
def test_step_replayed_as_a_graph(name, seqlen):
    wl = WORKLOADS[name]
    x = {k: v.cuda() for k, v in generate(wl, seqlen=seqlen).items()}
    mode = ops.SELECT_GLOBAL if wl.select_mode == "global" else ops.SELECT_BLOCK

    def step():
        idx = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, max_seqlen=seqlen,
                                   select_mode=mode, block_size=wl.block_size, stats_scope=ops.STATS_SEQUENCE)
        out, lse = ops.attention_forward(x["q"], x["k"], x["v"], x["w"], x["cu"], idx, None, max_seqlen=seqlen,
                                         select_mode=mode, block_size=wl.block_size)
        res = [idx, out, lse]
        if wl.backward:
            res += list(ops.attention_backward(x["dout"], x["q"], x["k"], x["v"], out, lse, x["w"], x["cu"], idx,
                                               max_seqlen=seqlen, want_dbias=False)[:3])
        return res

    ref = [t.clone() for t in step()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()  # torch's capture recipe: warm up on a side stream first
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for rep in range(3):
        for t in outs:  # clobber the graph's outputs so each replay has to rewrite them
            t.fill_(-1)
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(outs, ref)):
            assert torch.equal(a, b), (rep, i)
        eager = step()  # eager work between the replays
        torch.cuda.synchronize()
        for a, b in zip(eager, ref):
            assert torch.equal(a, b)


def test_two_streams_at_once():
    """Two independent steps enqueued on two streams (default priority) at the same time, each
    with its own workspaces, equal the same steps run one after the other."""
    wl = WORKLOADS["fwdbwd_bf16_h16_l32768"]
    xs = [{k: v.cuda() for k, v in generate(wl, seqlen=4096, heads=h).items()} for h in (16, 8)]

    def step(x):
        idx = ops.select_landmarks(x["h"], x["v"], x["alpha"], x["w"], x["cu"], wl.k_lmk, max_seqlen=4096,
                                   stats_scope=ops.STATS_SEQUENCE)
        out, lse = ops.attention_forward(x["q"], x["k"], x["v"], x["w"], x["cu"], idx, None, max_seqlen=4096)
        return [idx, out, lse] + list(ops.attention_backward(x["dout"], x["q"], x["k"], x["v"], out, lse, x["w"],
                                                             x["cu"], idx, max_seqlen=4096, want_dbias=False)[:3])

    ref = [[t.clone() for t in step(x)] for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    res = []
    for s, x in zip(streams, xs):
        with torch.cuda.stream(s):
            res.append(step(x))
    torch.cuda.synchronize()
    for r, e in zip(res, ref):
        for a, b in zip(r, e):
            assert torch.equal(a, b)
