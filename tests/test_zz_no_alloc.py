"""lcv_bsa_forward_noalloc (no workspace: the launch order in a fixed 1 MiB
device array, the pooled means and block scores staged in out) against
lcv_bsa_forward (caller workspace), through the C ABI.

Two calls in a row, the second on a smaller problem than the first, so the
second reads an array that still holds the first call's launch order:
routing must be identical and the output bit-identical (same attention
kernel, same routing, same launch order).  Also: an out in [B, S, H, D]
order, the sliced and the fused routing, two calls on two streams with no
synchronisation between them (the library orders them), graph capture, and
a problem beyond the array (refused with LCV_BSA_ERR_UNSUPPORTED; its
tensors are sized for it, so nothing would read out of bounds even if it
were not refused).
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


def _score_slices(B, H, nb, D, esz=2):
    """(heads per score slice, slices) of the no-allocation routing for a
    256-byte aligned out of B*H*nb*64*D elements of esz bytes; 0 slices
    means the fused select kernel routes."""
    r256 = lambda x: (x + 255) // 256 * 256  # noqa: E731
    left = B * H * nb * 64 * D * esz - 2 * r256(B * H * nb * D * 4)
    per = left // r256(nb * nb * 4)
    slices = -(-B * H // per) if per else 0
    return per, (slices if slices <= 8 else 0)


def _inputs(device, B, H, S, D, dtype, top_k, seed, grid):
    from lcv_bsa.workloads import make_inputs

    return make_inputs(B, H, D, (1, 1, S), (1, 1, 64), dtype, device, seed=seed, grid=grid,
                       margin_ks=(top_k,))[:3]


def _reference(device, lib, q, k, v, top_k):
    from lcv_bsa import _lib

    B, H, S, D = q.shape
    nb = S // 64
    ws = torch.empty((lib.lcv_bsa_forward_workspace_bytes(B, H, nb, D),), dtype=torch.uint8, device=device)
    out_ref, idx_ref = torch.empty_like(q), torch.empty((B, H, nb, top_k), dtype=torch.int32, device=device)
    _lib.check(_call(lib, "lcv_bsa_forward", q, k, v, top_k, (1, 1, S), (1, 1, 64), out_ref, idx_ref, ws),
               "forward")
    return out_ref, idx_ref


def _empty_out(q, layout):
    """out filled with NaN, as a [B, H, S, D] view of [B, H, S, D] or
    [B, S, H, D] storage."""
    B, H, S, D = q.shape
    if layout == "bhsd":
        return torch.full_like(q, float("nan"))
    return torch.full((B, S, H, D), float("nan"), dtype=q.dtype, device=q.device).permute(0, 2, 1, 3)


def _compare(device, lib, B, H, grid, D, dtype, top_k, seed, layout="bhsd", S=None):
    from lcv_bsa import _lib

    S = S or grid[0] * grid[1] * grid[2]
    nb = S // 64
    q, k, v = _inputs(device, B, H, S, D, dtype, top_k, seed, grid)
    out_ref, idx_ref = _reference(device, lib, q, k, v, top_k)
    out = _empty_out(q, layout)
    idx = torch.full((B, H, nb, top_k), -7, dtype=torch.int32, device=device)
    _lib.check(_call(lib, "lcv_bsa_forward_noalloc", q, k, v, top_k, (1, 1, S), (1, 1, 64), out, idx),
               "forward_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(idx, idx_ref), "routing differs"
    assert torch.equal(out, out_ref), "output differs"
    per, slices = _score_slices(B, H, nb, D)
    route = f"{slices} score slice(s) of {per} heads" if slices else "fused select"
    print(f"no-alloc B{B} H{H} S{S} D{D} {dtype} top-k {top_k} out {layout}, {route}: "
          "routing and output identical", flush=True)


def test_noalloc_matches_forward_twice_second_smaller(device):
    from lcv_bsa import _lib

    lib = _lib.load()
    # 720p headline shape first (every head's scores staged in out at once),
    # then a smaller problem.
    assert _score_slices(1, 32, 900, 128) == (136, 1)
    _compare(device, lib, 1, 32, (16, 45, 80), 128, torch.float16, 57, seed=31)
    _compare(device, lib, 1, 4, (2, 16, 64), 64, torch.bfloat16, 5, seed=32)


def test_noalloc_out_in_bshd_order(device):
    """out as a [B, H, S, D] view of [B, S, H, D] storage (the layout the DiT
    block's projection reads): dense, so the means and scores are staged in
    it; the result equals lcv_bsa_forward's into the same layout."""
    from lcv_bsa import _lib

    lib = _lib.load()
    _compare(device, lib, 2, 8, (4, 16, 64), 128, torch.float16, 9, seed=34, layout="bshd")


def test_noalloc_out_off_a_256_byte_boundary(device):
    """out 16 bytes past a 256-byte boundary (a view into a larger buffer):
    the means and scores are staged from the next 256-byte boundary inside
    out, and the bytes of the buffer outside out are left untouched."""
    from lcv_bsa import _lib

    lib = _lib.load()
    B, H, D, top_k, grid = 1, 8, 128, 9, (4, 16, 64)
    S = grid[0] * grid[1] * grid[2]
    nb = S // 64
    q, k, v = _inputs(device, B, H, S, D, torch.float16, top_k, 38, grid)
    out_ref, idx_ref = _reference(device, lib, q, k, v, top_k)
    n = B * H * S * D
    buf = torch.full((n + 256,), 7.0, dtype=torch.float16, device=device)
    assert buf.data_ptr() % 256 == 0
    out = buf[8:8 + n].view(B, H, S, D)  # 16 bytes past the boundary
    idx = torch.full((B, H, nb, top_k), -7, dtype=torch.int32, device=device)
    _lib.check(_call(lib, "lcv_bsa_forward_noalloc", q, k, v, top_k, (1, 1, S), (1, 1, 64), out, idx),
               "forward_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(idx, idx_ref), "routing differs"
    assert torch.equal(out, out_ref), "output differs"
    assert bool((buf[:8] == 7.0).all()) and bool((buf[8 + n:] == 7.0).all()), "bytes outside out changed"


def test_noalloc_refuses_beyond_scratch(device):
    from lcv_bsa import _lib

    lib = _lib.load()
    # B*H*nb = 5 * 64 * 900 = 288,000 > 262,144: a launch order beyond 1 MiB.
    B, H, S, D, top_k = 5, 64, 57600, 64, 57
    q = torch.zeros((B, H, S, D), dtype=torch.float16, device=device)
    out = torch.empty_like(q)
    idx = torch.empty((B, H, S // 64, top_k), dtype=torch.int32, device=device)
    st = _call(lib, "lcv_bsa_forward_noalloc", q, q, q, top_k, (1, 1, S), (1, 1, 64), out, idx)
    assert st == _lib.ERR_UNSUPPORTED
    assert b"fixed device scratch" in lib.lcv_bsa_last_error()
    st = _call(lib, "lcv_bsa_forward_noalloc", q, q, q, top_k, (1, 1, S), (1, 1, 64), q, idx)
    assert st == _lib.ERR_UNSUPPORTED  # the size check comes first


def test_noalloc_two_score_slices(device):
    """2048 blocks at D=64, 16 heads: out holds the scores of 15 heads, so the
    routing runs as two score GEMM + top-k slices."""
    from lcv_bsa import _lib

    lib = _lib.load()
    assert _score_slices(1, 16, 2048, 64) == (15, 2)
    _compare(device, lib, 1, 16, None, 64, torch.float16, 8, seed=35, S=2048 * 64)


def test_noalloc_fused_route_when_scores_do_not_fit(device):
    """2048 blocks at D=64, one head: one head's 16 MiB of scores do not fit
    beside the means in its 16 MiB out, so the fused select kernel routes
    (at num_blocks <= 2048 with the same split-bf16 MFMA scores)."""
    from lcv_bsa import _lib

    lib = _lib.load()
    assert _score_slices(1, 1, 2048, 64) == (0, 0)
    _compare(device, lib, 1, 1, None, 64, torch.bfloat16, 8, seed=33, S=2048 * 64)


def test_noalloc_calls_on_two_streams_are_ordered(device):
    """Two calls on two streams with no synchronisation between them: the
    second call's stream waits for the first call's work (both use the
    device's launch-order array), so each result equals lcv_bsa_forward's.
    Both problems have the same size, so every launch-order entry is in
    range for either call."""
    from lcv_bsa import _lib

    lib = _lib.load()
    B, H, D, top_k, grid = 1, 32, 128, 57, (16, 45, 80)
    S = grid[0] * grid[1] * grid[2]
    nb = S // 64
    a = _inputs(device, B, H, S, D, torch.float16, top_k, 36, grid)
    b = _inputs(device, B, H, S, D, torch.float16, top_k, 37, grid)
    ref_a, ref_b = _reference(device, lib, *a, top_k), _reference(device, lib, *b, top_k)
    outs = [torch.full_like(a[0], float("nan")) for _ in range(2)]
    idxs = [torch.full((B, H, nb, top_k), -7, dtype=torch.int32, device=device) for _ in range(2)]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=device) for _ in range(2)]
    for rep in range(3):
        for s, (q, k, v), o, i in zip(streams, (a, b), outs, idxs):
            with torch.cuda.stream(s):
                _lib.check(_call(lib, "lcv_bsa_forward_noalloc", q, k, v, top_k, (1, 1, S), (1, 1, 64), o, i),
                           "forward_noalloc")
        torch.cuda.synchronize()
        for (out_ref, idx_ref), o, i, name in zip((ref_a, ref_b), outs, idxs, "ab"):
            assert torch.equal(i, idx_ref), f"rep {rep} call {name}: routing"
            assert torch.equal(o, out_ref), f"rep {rep} call {name}: output"
            o.fill_(float("nan"))
        torch.cuda.synchronize()
    print("no-alloc on two streams: 3 x 2 calls equal the workspace results", flush=True)


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
