"""The operator under stream concurrency and HIP graph capture.

The library keeps no per-call state on the host or the device (the caller
owns every buffer), launches only on the stream it is given and never
synchronises, so:

* forwards queued on two streams at once give the same bits as the same
  forwards run one after the other;
* ``bsa_attention`` captured into a HIP graph (through torch's graph API)
  replays to the eager result every time -- also with eager work between
  the replays and after the captured inputs change in place.

All streams keep the default priority.  The routing and the launch order
are deterministic, so every comparison is bit-exact.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPE, CHUNK = (4, 16, 16), (4, 4, 4)  # 1024 tokens, 16 voxel blocks


def _inputs(device, seed, B=1, H=4, D=128, dtype=torch.float16):
    from lcv_bsa.workloads import make_inputs

    q, k, v, _ = make_inputs(B, H, D, SHAPE, CHUNK, dtype, device, seed=seed, margin_ks=(4,))
    return q, k, v


def _forward(q, k, v):
    from lcv_bsa import bsa_attention

    return bsa_attention(q, k, v, shape=SHAPE, chunk_thw=CHUNK, top_k=4, return_indices=True)


def test_two_streams_match_serial(device):
    cases = [_inputs(device, s) for s in (1, 2, 3, 4)]
    ref = [_forward(*c) for c in cases]
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream(device=device), torch.cuda.Stream(device=device)]
    got = [None] * len(cases)
    torch.cuda.synchronize()
    for rep in range(3):
        for i, c in enumerate(cases):
            s = streams[i % 2]
            s.wait_stream(torch.cuda.current_stream(device))
            with torch.cuda.stream(s):
                got[i] = _forward(*c)
        for s in streams:
            torch.cuda.current_stream(device).wait_stream(s)
        torch.cuda.synchronize()
        for i in range(len(cases)):
            assert torch.equal(got[i][0], ref[i][0]), f"output of case {i}, round {rep}"
            assert torch.equal(got[i][1], ref[i][1]), f"routing of case {i}, round {rep}"


def test_graph_capture_replays_eager_result(device):
    q, k, v = _inputs(device, 7)
    q2, _, _ = _inputs(device, 8)
    eager_out, eager_idx = _forward(q, k, v)
    eager2_out, eager2_idx = _forward(q2, k, v)
    torch.cuda.synchronize()

    # Warm up on a side stream, as torch's graph capture requires.
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        for _ in range(2):
            _forward(q, k, v)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out, idx = _forward(q, k, v)
    torch.cuda.synchronize()

    scratch = torch.randn(1 << 20, device=device)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out), f"replay {rep}: output"
        assert torch.equal(idx, eager_idx), f"replay {rep}: routing"
        scratch.mul_(1.5).add_(0.25)  # eager work between replays
        torch.cuda.synchronize()

    q.copy_(q2)  # new contents in the captured input buffer
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager2_out) and torch.equal(idx, eager2_idx), "replay after input change"
