"""GPU parity of the fused pre-BSA pass (lcv_bsa_prepare_qk) against the oracle.

q / k come in as the DiT produces them: [B, H, N, D] views of the fused QKV
projection output [B, N, 3, H, D] (attention.py:191-194).  The outputs must
match the oracle's RMSNorm_FP32 -> RoPE chain (blocks.py:55-72,
rope_3d.py:107-128) to one unit in the last place of the dtype (rsqrt and the
fp32 summation order may round differently), and the fused block means must
equal the pooling of the written q / k.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import assert_close_report
from oracle import bsa_oracle as O

pytestmark = pytest.mark.gpu

ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}
NAME = {torch.float16: "f16", torch.bfloat16: "bf16"}

# (rope grid, BSA shape, chunk)
GEOMS = [
    ((4, 16, 64), (1, 1, 4096), (1, 1, 64)),
    ((8, 8, 16), (8, 8, 16), (4, 4, 4)),
    ((2, 45, 32), (1, 1, 2880), (1, 1, 64)),
]


def _np(t):
    return t.detach().float().cpu().numpy()


def _qkv_views(B, N, H, D, dtype, device, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    qkv = (torch.randn(B, N, 3, H, D, generator=g) * 1.5 + 0.3).to(dtype).to(device)
    q = qkv[:, :, 0].transpose(1, 2)
    k = qkv[:, :, 1].transpose(1, 2)
    v = qkv[:, :, 2].transpose(1, 2)
    assert not q.is_contiguous() and q.stride(-1) == 1
    return q, k, v


def _pair_mag(y):
    """|u| + |v| of each element's RoPE pair (dims 2i, 2i+1)."""
    a = np.abs(y).reshape(*y.shape[:-1], y.shape[-1] // 2, 2).sum(-1)
    return np.repeat(a, 2, axis=-1)


def _check_ulp(got, ref, dtype, what, pre=None):
    """Almost every element within 1 ulp of the oracle; every element within
    one ulp of the RoPE pair's input magnitude (``pre``, the normalized values
    before RoPE): a 1-ulp difference in the normalized pair -- rsqrt rounding
    may flip one -- passes through x*cos - y*sin, which cancels near zero."""
    ulp = ULP[dtype]
    bound = ulp * np.maximum(np.abs(ref), 2.0 ** -14)
    err = np.abs(got - ref)
    bad = err > bound
    assert bad.mean() < 1e-3, f"{what}: {bad.mean():.2e} of elements beyond 1 ulp"
    wide = 2 * bound if pre is None else ulp * (np.abs(ref) + _pair_mag(pre)) + 2.0 ** -24
    assert np.all(err <= wide), f"{what}: max excess {np.max(err / wide):.2f} of the bound"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("grid,shape,chunk", GEOMS)
def test_prepare_matches_oracle(device, dtype, D, grid, shape, chunk):
    from lcv_bsa import prepare_qk

    N = int(np.prod(grid))
    q, k, _ = _qkv_views(1, N, 2, D, dtype, device, seed=N + D)
    g = torch.Generator(device="cpu").manual_seed(7)
    wq = (1.0 + 0.2 * torch.randn(D, generator=g)).to(dtype).to(device)
    wk = (1.0 + 0.2 * torch.randn(D, generator=g)).to(dtype).to(device)
    qo, ko, qb, kb = prepare_qk(q, k, grid, q_weight=wq, k_weight=wk, shape=shape, chunk_thw=chunk)
    assert qo.dtype == dtype and qo.is_contiguous() and qb.dtype == torch.float32
    rq, rk, rqb, rkb = O.prepare_qk(_np(q), _np(k), grid, shape, chunk, _np(wq), _np(wk), 1e-6, NAME[dtype])
    yq = O.rms_norm_fp32(_np(q), _np(wq), 1e-6, NAME[dtype])
    yk = O.rms_norm_fp32(_np(k), _np(wk), 1e-6, NAME[dtype])
    _check_ulp(_np(qo), rq, dtype, f"q {grid} D={D}", yq)
    _check_ulp(_np(ko), rk, dtype, f"k {grid} D={D}", yk)
    # The fused means are the block means of what was written.
    assert_close_report(_np(qb), O.mean_pool_blocks_3d(_np(qo), shape, chunk), 1e-5, 1e-6, "q means")
    assert_close_report(_np(kb), O.mean_pool_blocks_3d(_np(ko), shape, chunk), 1e-5, 1e-6, "k means")
    assert_close_report(_np(qb), rqb, 4 * ULP[dtype], ULP[dtype] / 8, "q means vs oracle")


def test_prepare_default_weight_and_eps(device):
    from lcv_bsa import prepare_qk

    q, k, _ = _qkv_views(1, 1024, 1, 128, torch.float16, device, seed=3)
    q = q * 1e-3  # small rows: eps matters
    qo, _, _, _ = prepare_qk(q, k, (8, 8, 16), eps=1e-2, shape=(8, 8, 16), chunk_thw=(4, 4, 4))
    rq, _, _, _ = O.prepare_qk(_np(q), _np(k), (8, 8, 16), (8, 8, 16), (4, 4, 4), None, None, 1e-2, "f16")
    _check_ulp(_np(qo), rq, torch.float16, "default weight, eps 1e-2", O.rms_norm_fp32(_np(q), None, 1e-2, "f16"))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_bsa_from_prepared_means(device, dtype):
    """bsa_attention(..., block_means=prepare_qk means): routing is the exact
    top-k of the fp64 scores of those means, and the output matches the
    oracle's attention over that routing."""
    from lcv_bsa import bsa_attention, prepare_qk

    grid, shape, chunk = (4, 16, 64), (1, 1, 4096), (1, 1, 64)
    q, k, v = _qkv_views(1, 4096, 2, 128, dtype, device, seed=11)
    qo, ko, qb, kb = prepare_qk(q, k, grid, shape=shape, chunk_thw=chunk)
    out, idx = bsa_attention(qo, ko, v, shape, sparsity=0.9375, chunk_thw=chunk,
                             return_indices=True, block_means=(qb, kb))
    ref_idx, _ = O.topk_block_indices(O.block_routing_scores(_np(qb), _np(kb)), top_k=idx.shape[-1])
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    ref = O.sparse_attention_from_indices(_np(qo), _np(ko), _np(v), ref_idx, shape, chunk)
    tol = {torch.float16: (2e-3, 2e-4), torch.bfloat16: (1e-2, 2e-3)}[dtype]
    assert_close_report(_np(out), ref, *tol, f"bsa from prepared {dtype}")


def test_prepare_rejects_bad_arguments(device):
    from lcv_bsa import prepare_qk

    q, k, _ = _qkv_views(1, 1024, 1, 128, torch.float16, device, seed=5)
    with pytest.raises(ValueError, match="multiple of"):
        prepare_qk(q, k, (8, 8, 16), shape=(8, 8, 16), chunk_thw=(4, 4, 3))
    with pytest.raises(ValueError, match="RoPE grid"):
        prepare_qk(q, k, (8, 8, 8), shape=(8, 8, 16), chunk_thw=(4, 4, 4))
    with pytest.raises(ValueError):
        prepare_qk(q.float(), k.float(), (8, 8, 16), shape=(8, 8, 16), chunk_thw=(4, 4, 4))
    with pytest.raises(ValueError, match="norm weight"):
        prepare_qk(q, k, (8, 8, 16), q_weight=torch.ones(64, device=device), shape=(8, 8, 16),
                   chunk_thw=(4, 4, 4))
