"""lcv_bsa_forward_noalloc (no workspace, fixed device scratch) against
lcv_bsa_forward (caller workspace), through the C ABI.

Two calls in a row, the second on a smaller problem than the first, so the
second reads a scratch array that still holds the first call's means and
launch order: routing must be identical and the output bit-identical (same
attention kernel, same routing, same launch order).  A problem beyond the
scratch is refused with LCV_BSA_ERR_UNSUPPORTED (its tensors are sized for
it, so nothing would read out of bounds even if it were not refused).
"""

from __future__ import annotations

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def _call(lib, fn, q, k, v, top_k, shape, chunk, out, idx, ws=None):
    from lcv_bsa import _lib
    from lcv_bsa.block_sparse_attention import _geom, _strides

    B, H, S, D = q.shape
    code = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}[q.dtype]
    stream = torch.cuda.current_stream(q.device).cuda_stream
    args = [q.data_ptr(), k.data_ptr(), v.data_ptr(), code, B, H, S, D, _strides(q), _strides(k), _strides(v),
            top_k, 1.0 / math.sqrt(D), _geom(shape, chunk)]
    if fn == "lcv_bsa_forward":
        args += [ws.data_ptr(), ws.numel()]
    args += [idx.data_ptr(), out.data_ptr(), _strides(out), stream]
    return getattr(lib, fn)(*args)


def _compare(device, lib, B, H, grid, D, dtype, top_k, seed):
    from lcv_bsa import _lib
    from lcv_bsa.workloads import make_inputs

    S = grid[0] * grid[1] * grid[2]
    shape, chunk = (1, 1, S), (1, 1, 64)
    nb = S // 64
    q, k, v, _ = make_inputs(B, H, D, shape, chunk, dtype, device, seed=seed, grid=grid, margin_ks=(top_k,))
    ws = torch.empty((lib.lcv_bsa_forward_workspace_bytes(B, H, nb, D),), dtype=torch.uint8, device=device)
    out_ref, idx_ref = torch.empty_like(q), torch.empty((B, H, nb, top_k), dtype=torch.int32, device=device)
    _lib.check(_call(lib, "lcv_bsa_forward", q, k, v, top_k, shape, chunk, out_ref, idx_ref, ws), "forward")
    out = torch.full_like(q, float("nan"))
    idx = torch.full((B, H, nb, top_k), -7, dtype=torch.int32, device=device)
    _lib.check(_call(lib, "lcv_bsa_forward_noalloc", q, k, v, top_k, shape, chunk, out, idx), "forward_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(idx, idx_ref), "routing differs"
    assert torch.equal(out, out_ref), "output differs"
    print(f"no-alloc B{B} H{H} S{S} D{D} {dtype} top-k {top_k}: routing and output identical", flush=True)


def test_noalloc_matches_forward_twice_second_smaller(device):
    from lcv_bsa import _lib

    lib = _lib.load()
    # 720p headline shape first (29.6 MB of scratch), then a smaller problem.
    _compare(device, lib, 1, 32, (16, 45, 80), 128, torch.float16, 57, seed=31)
    _compare(device, lib, 1, 4, (2, 16, 64), 64, torch.bfloat16, 5, seed=32)


def test_noalloc_refuses_beyond_scratch(device):
    from lcv_bsa import _lib

    lib = _lib.load()
    # B*H*nb = 2 * 64 * 900 = 115,200 > 65,280: 118 MB of means and order.
    B, H, S, D, top_k = 2, 64, 57600, 128, 57
    q = torch.zeros((B, H, S, D), dtype=torch.float16, device=device)
    out = torch.empty_like(q)
    idx = torch.empty((B, H, S // 64, top_k), dtype=torch.int32, device=device)
    st = _call(lib, "lcv_bsa_forward_noalloc", q, q, q, top_k, (1, 1, S), (1, 1, 64), out, idx)
    assert st == _lib.ERR_UNSUPPORTED
    assert b"fixed device scratch" in lib.lcv_bsa_last_error()


def test_noalloc_fused_route_when_score_slices_do_not_fit(device):
    """56 heads at 720p leave scratch for 4 heads of block scores: 14 slices,
    more than the sliced route takes, so the fused select kernel routes."""
    from lcv_bsa import _lib

    lib = _lib.load()
    _compare(device, lib, 1, 56, (16, 45, 80), 128, torch.float16, 57, seed=33)


def test_noalloc_graph_capture_replays_eager(device):
    """lcv_bsa_forward_noalloc captured into a HIP graph (after an eager call
    on the device resolved the scratch address) replays to the eager bits --
    with eager no-allocation calls on other inputs between the replays, which
    rewrite the shared scratch, and after the captured input changes in
    place."""
    from lcv_bsa import _lib
    from lcv_bsa.workloads import make_inputs

    lib = _lib.load()
    B, H, D, top_k, grid = 1, 4, 128, 4, (4, 16, 64)
    S = grid[0] * grid[1] * grid[2]
    shape, chunk, nb = (1, 1, S), (1, 1, 64), S // 64
    q, k, v, _ = make_inputs(B, H, D, shape, chunk, torch.float16, device, seed=41, grid=grid, margin_ks=(top_k,))
    q2, k2, v2, _ = make_inputs(B, H, D, shape, chunk, torch.float16, device, seed=42, grid=grid, margin_ks=(top_k,))

    def run(qq, kk, vv):
        o = torch.empty_like(qq)
        i = torch.empty((B, H, nb, top_k), dtype=torch.int32, device=device)
        _lib.check(_call(lib, "lcv_bsa_forward_noalloc", qq, kk, vv, top_k, shape, chunk, o, i), "noalloc")
        return o, i

    eager_out, eager_idx = run(q, k, v)
    eager2_out, eager2_idx = run(q2, k, v)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        run(q, k, v)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize()

    out = torch.empty_like(q)
    idx = torch.empty((B, H, nb, top_k), dtype=torch.int32, device=device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = _call(lib, "lcv_bsa_forward_noalloc", q, k, v, top_k, shape, chunk, out, idx)
    assert st == 0, lib.lcv_bsa_last_error()
    torch.cuda.synchronize()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager_out), f"replay {rep}: output"
        assert torch.equal(idx, eager_idx), f"replay {rep}: routing"
        other_out, _ = run(q2, k2, v2)  # eager call in between: rewrites the scratch
        torch.cuda.synchronize()
    q.copy_(q2)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, eager2_out) and torch.equal(idx, eager2_idx), "replay after input change"
    print("no-alloc graph: 4 replays equal the eager results", flush=True)


_FIRST_CALL_UNDER_CAPTURE = r"""
import math, sys, torch
sys.path[:0] = [{repo!r}, {pkg!r}]
from lcv_bsa import _lib
from lcv_bsa.block_sparse_attention import _geom, _strides
from lcv_bsa.workloads import make_inputs
lib = _lib.load()
dev = torch.device("cuda", 0)
B, H, D, top_k, grid = 1, 2, 64, 3, (2, 16, 64)
S = grid[0] * grid[1] * grid[2]
shape, chunk, nb = (1, 1, S), (1, 1, 64), S // 64
q, k, v, _ = make_inputs(B, H, D, shape, chunk, torch.bfloat16, dev, seed=5, grid=grid, margin_ks=(top_k,))
out = torch.empty_like(q)
idx = torch.empty((B, H, nb, top_k), dtype=torch.int32, device=dev)
def call():
    s = torch.cuda.current_stream(dev).cuda_stream
    return lib.lcv_bsa_forward_noalloc(q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.BF16, B, H, S, D,
        _strides(q), _strides(k), _strides(v), top_k, 1.0 / math.sqrt(D), _geom(shape, chunk),
        idx.data_ptr(), out.data_ptr(), _strides(out), s)
pad = torch.zeros(16, device=dev)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    pad.add_(1.0)
    st = call()
assert st == _lib.ERR_UNSUPPORTED, st
assert b"under stream capture" in lib.lcv_bsa_last_error(), lib.lcv_bsa_last_error()
assert call() == 0  # eager: resolves the address
torch.cuda.synchronize()
ref_out, ref_idx = out.clone(), idx.clone()
out.zero_(); idx.zero_()
g2 = torch.cuda.CUDAGraph()
with torch.cuda.graph(g2):
    st = call()
assert st == 0, lib.lcv_bsa_last_error()
g2.replay()
torch.cuda.synchronize()
assert torch.equal(out, ref_out) and torch.equal(idx, ref_idx)
print("child ok")
"""


def test_noalloc_first_call_under_capture_is_refused(device):
    """In a fresh process, a first call on the device made under stream
    capture is refused with LCV_BSA_ERR_UNSUPPORTED before any device work;
    after one eager call, a captured call works and replays to its result."""
    import subprocess
    import sys
    from pathlib import Path

    repo = Path(__file__).resolve().parents[1]
    code = _FIRST_CALL_UNDER_CAPTURE.format(repo=str(repo), pkg=str(repo / "longcat-video-mlx_amd"))
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], r.stderr[-2000:])
    assert r.returncode == 0 and "child ok" in r.stdout
