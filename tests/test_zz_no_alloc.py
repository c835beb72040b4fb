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
