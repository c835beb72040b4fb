"""GPU parity of each native kernel against the oracle, through the C ABI.

Mirrors the reference's kernel gates (tests/smoke/test_bsa_tier_b_smoke.py)
and adds exact checks for the integer/index work.  Tolerances (attention
output vs the fp64 oracle on the same, already-rounded inputs):
  fp16 : max-abs 2e-3, mean-abs 2e-4
  bf16 : max-abs 1e-2, mean-abs 2e-3 (P and the output carry 8-bit mantissas)
  fp32 : max-abs 2e-5, mean-abs 2e-6
Block indices, token maps, masks and permutations must be bit-exact.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import assert_close_report, wide_range_inputs
from oracle import bsa_oracle as O

pytestmark = pytest.mark.gpu

TOL = {
    torch.float16: (2e-3, 2e-4),
    torch.bfloat16: (1e-2, 2e-3),
    torch.float32: (2e-5, 2e-6),
}


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy() if t.dtype != torch.float64 else t.cpu().numpy()


def _rand(shape, dtype, device, seed):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype).to(device)


def _distinct_indices(B, H, nq, nk, k, seed, sort=True):
    rng = np.random.default_rng(seed)
    out = np.empty((B, H, nq, k), dtype=np.int32)
    for b in range(B):
        for h in range(H):
            for i in range(nq):
                sel = rng.choice(nk, size=k, replace=False)
                out[b, h, i] = np.sort(sel) if sort else sel
    return out


def test_library_version(device):
    from lcv_bsa import _lib

    v = _lib.version()
    print("library:", v)
    assert "gfx950" in v


# ---------------------------------------------------------------------------
# Pooling (block_sparse_attention.py:67-104)
# ---------------------------------------------------------------------------

POOL_CASES = [
    ((1, 1, 4096), (1, 1, 64), 64),
    ((8, 12, 16), (4, 4, 4), 128),
    ((4, 8, 8), (2, 2, 2), 32),
    ((8, 8, 8), (4, 4, 4), 4),
    ((2, 6, 10), (1, 2, 5), 24),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape,chunk,D", POOL_CASES)
def test_pool_matches_oracle(device, dtype, shape, chunk, D):
    from lcv_bsa import mean_pool_blocks_3d

    S = int(np.prod(shape))
    x = _rand((2, 3, S, D), dtype, device, seed=S + D)
    got = mean_pool_blocks_3d(x, shape, chunk)
    ref = O.mean_pool_blocks_3d(_np(x), shape, chunk)
    assert got.dtype == torch.float32
    assert_close_report(_np(got), ref, 2e-6, 2e-7, f"pool {shape} {chunk} D={D} {dtype}")


def test_pool_strided_view(device):
    """q as the DiT produces it: a [B,H,S,D] view of a [B,S,H,D] buffer."""
    from lcv_bsa import mean_pool_blocks_3d

    base = _rand((1, 4096, 4, 128), torch.float16, device, seed=5)
    x = base.transpose(1, 2)
    assert not x.is_contiguous() and x.stride(3) == 1
    got = mean_pool_blocks_3d(x, (1, 1, 4096), (1, 1, 64))
    ref = O.mean_pool_blocks_3d(_np(x.contiguous()), (1, 1, 4096), (1, 1, 64))
    assert_close_report(_np(got), ref, 2e-6, 2e-7, "pool strided")


def test_pool_rejects_bad_shape(device):
    from lcv_bsa import mean_pool_blocks_3d

    x = torch.zeros((1, 1, 96, 8), device=device)
    with pytest.raises(ValueError, match="multiple of"):
        mean_pool_blocks_3d(x, (4, 4, 6), (4, 4, 4))
    with pytest.raises(ValueError, match="doesn't match"):
        mean_pool_blocks_3d(torch.zeros((1, 1, 100, 8), device=device), (4, 4, 4))


# ---------------------------------------------------------------------------
# Scores and top-k (block_sparse_attention.py:107-134)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("nq,nk,D", [(1, 1, 4), (7, 63, 16), (64, 64, 64), (65, 65, 128),
                                     (100, 900, 128), (33, 2049, 32), (5, 4096, 8)])
def test_scores_match_oracle(device, nq, nk, D):
    from lcv_bsa import block_routing_scores

    qb = _rand((2, 2, nq, D), torch.float32, device, seed=nq)
    kb = _rand((2, 2, nk, D), torch.float32, device, seed=nk + 1)
    got = _np(block_routing_scores(qb, kb))
    ref = O.block_routing_scores(_np(qb), _np(kb))
    assert_close_report(got, ref, 2e-5 * math.sqrt(D), 2e-6 * math.sqrt(D), f"scores {nq}x{nk}x{D}")


@pytest.mark.parametrize("nq,nk,D", [(900, 900, 128), (450, 450, 64), (65, 2049, 128)])
def test_scores_error_within_piece_bound(device, nq, nk, D):
    """The bf16-piece GEMM drops only piece products below 2^-21 |x y|
    together and accumulates in fp32: against fp64, every score is within
    2e-6 of sum_d |x_d y_d|.  Dropping one kept product (2^-8 |x y|) or
    truncating an operand to bf16 would miss by three orders of magnitude."""
    from lcv_bsa import block_routing_scores

    qb = _rand((1, 2, nq, D), torch.float32, device, seed=11 * nq) * 0.7 + 0.2
    kb = _rand((1, 2, nk, D), torch.float32, device, seed=13 * nk) * 0.4 - 0.1
    got = block_routing_scores(qb, kb).double()
    q64, k64 = qb.double(), kb.double()
    ref = torch.matmul(q64, k64.transpose(-1, -2))
    env = torch.matmul(q64.abs(), k64.abs().transpose(-1, -2))
    ratio = ((got - ref).abs() / env).max().item()
    print(f"scores {nq}x{nk}x{D}: max |err| / envelope = {ratio:.2e}")
    assert ratio <= 2e-6


@pytest.mark.parametrize("nq", [131072 + 200, 262144 + 72])
def test_scores_large_head_offsets(device, nq):
    """One head whose score matrix passes 2^31 bytes (nq x 4096 keys): 2.2 GB
    and 4.3 GB.  Each 128-row tile writes through its own buffer resource, so
    the padding rows of the last tile cannot land on a real score and no
    offset wraps.  Rows at the start, around element 2^29 (byte 2^31), around
    element 2^30 (byte 2^32) where present, and at the end are checked
    against fp64 within the piece bound."""
    from lcv_bsa import block_routing_scores

    nk, D = 4096, 64
    qb = _rand((1, 1, nq, D), torch.float32, device, seed=5) * 0.7 + 0.2
    kb = _rand((1, 1, nk, D), torch.float32, device, seed=6) * 0.4 - 0.1
    got = block_routing_scores(qb, kb)
    torch.cuda.synchronize()
    rows = [0, 1, 127, 128, 131071, 131072, 131073, 131199, nq - 200, nq - 73, nq - 72, nq - 1]
    if nq > 262144:
        rows += [262143, 262144]
    rows = sorted({r for r in rows if 0 <= r < nq})
    sel = torch.tensor(rows, device=device)
    g = got[0, 0, sel].double().cpu()
    q64, k64 = qb[0, 0, sel].double().cpu(), kb[0, 0].double().cpu()
    ref = q64 @ k64.T
    env = q64.abs() @ k64.abs().T
    ratio = ((g - ref).abs() / env).max().item()
    print(f"scores nq={nq} nk={nk}: rows {rows[:3]}..{rows[-2:]} max |err| / envelope = {ratio:.2e}")
    assert ratio <= 2e-6
    del got


def test_scores_nonfinite_like_fp32(device):
    """inf / NaN in the pooled means: every score is NaN, +inf or -inf exactly
    where the fp32 GEMM's is (an inf meets no zero piece of the other
    operand), the finite ones stay within fp32 rounding, and the fused
    routing still equals scores + top-k."""
    from lcv_bsa import block_routing_scores, select_block_indices, topk_block_indices

    torch.backends.cuda.matmul.allow_tf32 = False
    for nq, nk, D, k in [(100, 300, 128, 19), (70, 200, 64, 12), (33, 129, 128, 64)]:
        qb = _rand((1, 2, nq, D), torch.float32, device, seed=nq)
        kb = _rand((1, 2, nk, D), torch.float32, device, seed=nk)
        qb[0, 0, 3, 5] = float("inf")
        qb[0, 0, 7, 9] = float("-inf")
        qb[0, 0, 11, 2] = float("nan")
        qb[0, 0, 13, 4], qb[0, 0, 13, 6] = float("inf"), float("-inf")
        kb[0, 0, 17, 8] = float("inf")
        kb[0, 0, 20, 1] = float("nan")
        kb[0, 1, 40, 3] = float("-inf")
        got = block_routing_scores(qb, kb)
        ref = torch.matmul(qb, kb.transpose(-1, -2))
        for cls in (torch.isnan, torch.isposinf, torch.isneginf):
            assert torch.equal(cls(got), cls(ref)), (nq, nk, D, cls.__name__)
        fin = torch.isfinite(ref)
        assert (got[fin] - ref[fin]).abs().max().item() <= 2e-5 * math.sqrt(D)
        two, _ = topk_block_indices(got, 0.0, top_k=k)
        assert torch.equal(select_block_indices(qb, kb, k, fused=True), two)


def test_scores_known_answer(device):
    """test_bsa_tier_a_smoke.py:68-75."""
    from lcv_bsa import block_routing_scores

    s = block_routing_scores(torch.ones((1, 1, 4, 8), device=device),
                             2 * torch.ones((1, 1, 4, 8), device=device))
    assert s.shape == (1, 1, 4, 4) and float(s[0, 0, 0, 0]) == 16.0


@pytest.mark.parametrize("nk", [1, 5, 64, 65, 127, 450, 900, 2048, 4096])
def test_topk_exact_with_ties(device, nk):
    """Integer-valued scores: many exact ties, resolved toward the lower index."""
    from lcv_bsa import topk_block_indices

    rng = np.random.default_rng(nk)
    sc = rng.integers(-20, 21, size=(2, 3, 17, nk)).astype(np.float32)
    sc[0, 0, 0] = -0.0
    sc[0, 0, 1] = np.nan
    sc[0, 0, 2, ::2] = np.nan
    sc[0, 0, 3] = -np.inf
    sc[0, 0, 4, :nk // 2] = np.inf
    sct = torch.from_numpy(sc).to(device)
    for k in sorted({1, max(1, nk // 16), max(1, nk // 2), nk}):
        got, kk = topk_block_indices(sct, 0.0, top_k=k)
        ref, _ = O.topk_block_indices(sc, top_k=k)
        assert kk == k
        assert np.array_equal(got.cpu().numpy(), ref), f"nk={nk} k={k}"


@pytest.mark.parametrize("nk", [64, 128, 129, 900, 2048])
def test_topk_lower_bound_paths(device, nk):
    """k on both sides of 64 and 128: the search over the keys above a lower
    bound (the smallest of the lanes' largest keys for k <= 64, of their
    second-largest keys for k <= 128) and the full search, on continuous
    scores and with a third of some rows tied at the top."""
    from lcv_bsa import topk_block_indices

    rng = np.random.default_rng(100 + nk)
    sc = rng.standard_normal((1, 2, 9, nk)).astype(np.float32)
    sc[0, 1, :3, : nk // 3] = 5.0
    sct = torch.from_numpy(sc).to(device)
    for k in sorted({1, 2, 57, 63, 64, 65, 100, 127, 128, 129} & set(range(1, nk + 1))):
        got, _ = topk_block_indices(sct, 0.0, top_k=k)
        ref, _ = O.topk_block_indices(sc, top_k=k)
        assert np.array_equal(got.cpu().numpy(), ref), f"nk={nk} k={k}"


@pytest.mark.parametrize("nk", [64, 900, 2048])
def test_topk_shared_prefix_rows(device, nk):
    """Rows whose candidate keys share long leading bit runs, where the
    search starts far below bit 31: one exponent (30 + small steps), values
    a few ulps apart, all-negative rows, and rows equal but for a few
    columns."""
    from lcv_bsa import topk_block_indices

    rng = np.random.default_rng(300 + nk)
    rows = []
    rows.append(30.0 + rng.random(nk))                                     # one exponent
    rows.append(np.float32(30.0) + rng.integers(0, 64, nk) * np.float32(2.0 ** -18))  # few-ulp steps
    rows.append(-1.0 - rng.random(nk))                                     # all negative, one exponent
    rows.append(-(2.0 ** -20) * (1 + rng.integers(0, 8, nk)))              # tiny negatives
    r = np.full(nk, 3.25)
    r[rng.integers(0, nk, 5)] = 3.5                                        # equal but for a few
    rows.append(r)
    rows.append(np.float32(1.0) + np.arange(nk) * np.float32(2.0 ** -23))  # consecutive floats
    sc = np.stack(rows).astype(np.float32)[None, None]
    sct = torch.from_numpy(sc).to(device)
    for k in sorted({1, 5, 6, 29, 57, 63, 64, 65, 113, 128} & set(range(1, nk + 1))):
        got, _ = topk_block_indices(sct, 0.0, top_k=k)
        ref, _ = O.topk_block_indices(sc, top_k=k)
        assert np.array_equal(got.cpu().numpy(), ref), f"nk={nk} k={k}"


def test_topk_count_rule(device):
    """test_bsa_tier_a_smoke.py:78-94 on the HIP top-k."""
    from lcv_bsa import topk_block_indices

    idx, n = topk_block_indices(_rand((1, 2, 4, 8), torch.float32, device, 1), sparsity=0.75)
    assert n == 2 and idx.shape == (1, 2, 4, 2)
    a = idx.cpu().numpy()
    assert (a >= 0).all() and (a < 8).all()
    _, n1 = topk_block_indices(_rand((1, 1, 2, 4), torch.float32, device, 2), sparsity=0.99)
    assert n1 == 1


@pytest.mark.parametrize("nq,nk,D,k", [(64, 64, 64, 4), (450, 450, 128, 29), (900, 900, 128, 57),
                                       (17, 1000, 16, 999), (3, 3000, 128, 187)])
def test_select_fused_equals_two_step(device, nq, nk, D, k):
    """Fused routing == scores + top-k (same fp32 products), and == the oracle
    on integer-valued means (exact in fp32, exact ties)."""
    from lcv_bsa import block_routing_scores, select_block_indices, topk_block_indices

    qb = _rand((1, 2, nq, D), torch.float32, device, seed=3 * nq)
    kb = _rand((1, 2, nk, D), torch.float32, device, seed=5 * nk)
    fused = select_block_indices(qb, kb, k, fused=True)
    two, _ = topk_block_indices(block_routing_scores(qb, kb), 0.0, top_k=k)
    assert torch.equal(fused, two)
    assert torch.equal(select_block_indices(qb, kb, k), two)
    qi, ki = torch.round(qb * 2), torch.round(kb * 2)
    ref, _ = O.topk_block_indices(O.block_routing_scores(_np(qi), _np(ki)), top_k=k)
    for f in (True, False):
        assert np.array_equal(select_block_indices(qi, ki, k, fused=f).cpu().numpy(), ref)


# ---------------------------------------------------------------------------
# Sparse attention from given indices (block_sparse_attention_metal.py contract)
# ---------------------------------------------------------------------------

ATTN_GEOMS = [
    ((1, 1, 512), (1, 1, 64)),
    ((8, 8, 16), (4, 4, 4)),
    ((2, 12, 16), (1, 4, 16)),
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("geom", ATTN_GEOMS)
def test_attn_matches_oracle(device, dtype, D, geom):
    from lcv_bsa import bsa_attention_hip

    shape, chunk = geom
    S = int(np.prod(shape))
    nb = S // 64
    B, H = 2, 2
    q, k, v = (_rand((B, H, S, D), dtype, device, seed=s) for s in (11, 12, 13))
    for topk in sorted({1, 3, nb}):
        idx = _distinct_indices(B, H, nb, nb, topk, seed=topk, sort=(topk != 3))
        out = bsa_attention_hip(q, k, v, torch.from_numpy(idx).to(device), chunk, shape)
        ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx, shape, chunk)
        assert out.dtype == dtype
        assert_close_report(_np(out), ref, *TOL[dtype], f"attn {dtype} D={D} {geom} k={topk}")


@pytest.mark.parametrize("dtype,topk", [(torch.float16, 129), (torch.bfloat16, 100)])
def test_attn_lists_longer_than_64(device, dtype, topk):
    """Routing lists of more than 64 entries: the tile walk reads them in
    64-entry chunks and starts each q-block's walk at a launch-slot-dependent
    entry, so with 8 heads x 130 q-blocks (1040 workgroups) the start lands
    in the second chunk for some of them and the walk wraps around.  Some
    rows carry padding (-1) in the second chunk and some are unsorted."""
    from lcv_bsa import bsa_attention_hip

    H, nb, D = 8, 130, 128
    S = nb * 64
    shape, chunk = (1, 1, S), (1, 1, 64)
    q, k, v = (_rand((1, H, S, D), dtype, device, seed=s) for s in (51, 52, 53))
    rng = np.random.default_rng(topk)
    idx = _distinct_indices(1, H, nb, nb, topk, seed=topk)
    for h in range(H):
        for r in rng.choice(nb, 6, replace=False):
            idx[0, h, r, 70 + rng.integers(0, topk - 70):] = -1  # padding in the second chunk
        for r in rng.choice(nb, 6, replace=False):
            rng.shuffle(idx[0, h, r])  # the walk does not rely on order for correctness
    out = bsa_attention_hip(q, k, v, torch.from_numpy(idx).to(device), chunk, shape)
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx, shape, chunk)
    assert_close_report(_np(out), ref, *TOL[dtype], f"attn top-k {topk} > 64 {dtype}")


@pytest.mark.parametrize("D", [16, 32, 256])
def test_attn_valu_head_dims(device, D):
    from lcv_bsa import bsa_attention_hip

    shape, chunk = (1, 1, 256), (1, 1, 64)
    q, k, v = (_rand((1, 2, 256, D), torch.float16, device, seed=s) for s in (1, 2, 3))
    idx = _distinct_indices(1, 2, 4, 4, 2, seed=D)
    out = bsa_attention_hip(q, k, v, torch.from_numpy(idx).to(device), chunk, shape)
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx, shape, chunk)
    assert_close_report(_np(out), ref, *TOL[torch.float16], f"attn valu D={D}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_attn_single_block_equals_dense(device, dtype):
    """test_bsa_tier_b_smoke.py:47-79 / :388-433: one block, top_k=1 == dense SDPA."""
    from lcv_bsa import bsa_attention_hip

    D = 128 if dtype == torch.float16 else 16
    q, k, v = (_rand((1, 2, 64, D), dtype, device, seed=s) for s in (0, 1, 2))
    out = bsa_attention_hip(q, k, v, torch.zeros((1, 2, 1, 1), dtype=torch.int32, device=device),
                            (4, 4, 4), (4, 4, 4))
    dense = torch.nn.functional.scaled_dot_product_attention(
        q.float().cpu(), k.float().cpu(), v.float().cpu(), scale=1.0 / math.sqrt(D))
    assert_close_report(_np(out), dense.numpy(), *TOL[dtype], f"single block {dtype}")


def test_attn_padding_and_duplicates(device):
    from lcv_bsa import bsa_attention_hip

    shape, chunk = (1, 1, 256), (1, 1, 64)
    q, k, v = (_rand((1, 1, 256, 128), torch.float16, device, seed=s) for s in (4, 5, 6))
    idx = np.array([[[[0, -1, 2], [1, 1, 3], [-1, -1, -1], [7, 3, 0]]]], dtype=np.int32)
    out = bsa_attention_hip(q, k, v, torch.from_numpy(idx).to(device), chunk, shape)
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx, shape, chunk)
    assert_close_report(_np(out), ref, *TOL[torch.float16], "padding/duplicates")
    assert (out[0, 0, 128:192] == 0).all()


def test_attn_strided_views_and_determinism(device):
    from lcv_bsa import bsa_attention_hip

    S, H, D = 1024, 4, 128
    buf = _rand((3, 1, S, H, D), torch.float16, device, seed=9)
    q, k, v = (buf[i].transpose(1, 2) for i in range(3))  # [1,H,S,D] views, stride(3)==1
    idx = torch.from_numpy(_distinct_indices(1, H, 16, 16, 5, seed=9)).to(device)
    o1 = bsa_attention_hip(q, k, v, idx, (1, 1, 64), (1, 1, S))
    o2 = bsa_attention_hip(q.contiguous(), k.contiguous(), v.contiguous(), idx, (1, 1, 64), (1, 1, S))
    assert torch.equal(o1, o2)
    o3 = bsa_attention_hip(q, k, v, idx, (1, 1, 64), (1, 1, S))
    assert torch.equal(o1, o3)


def test_attn_contract_errors(device):
    """test_bsa_tier_b_smoke.py:163-175 and the shape=None rule."""
    from lcv_bsa import bsa_attention_hip

    z = torch.zeros((1, 1, 48, 16), device=device)
    bi = torch.zeros((1, 1, 1, 1), dtype=torch.int32, device=device)
    with pytest.raises(ValueError, match="multiple of"):
        bsa_attention_hip(z, z, z, bi, (4, 4, 4), (4, 4, 4))
    z64 = torch.zeros((1, 1, 64, 16), device=device)
    with pytest.raises(ValueError, match="shape"):
        bsa_attention_hip(z64, z64, z64, bi, (4, 4, 4), None)
    z8 = torch.zeros((1, 1, 8, 16), device=device)
    with pytest.raises(ValueError, match="block_size=64"):
        bsa_attention_hip(z8, z8, z8, bi, (2, 2, 2), (2, 2, 2))
    z24 = torch.zeros((1, 1, 64, 24), device=device)
    with pytest.raises(ValueError, match="head_dim"):
        bsa_attention_hip(z24, z24, z24, bi, (4, 4, 4), (4, 4, 4))


# ---------------------------------------------------------------------------
# Index / layout helpers (exact)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape,chunk", [((4, 4, 4), (4, 4, 4)), ((8, 4, 4), (4, 4, 4)),
                                         ((6, 8, 12), (2, 4, 3)), ((1, 1, 57600), (1, 1, 64))])
def test_token_blocks_exact(device, shape, chunk):
    from lcv_bsa import build_token_block_indices

    got = build_token_block_indices(shape, chunk, device=device).cpu().numpy()
    assert np.array_equal(got, O.build_token_block_indices(shape, chunk))


def test_token_pair_mask_exact(device):
    from lcv_bsa import build_token_block_indices, build_token_pair_mask

    # the reference's known answer, test_bsa_tier_a_smoke.py:114-138
    bi = np.array([[[[3, 5], [0, 7]]]], dtype=np.int32)
    tbi = np.arange(8, dtype=np.int32)
    got = build_token_pair_mask(torch.from_numpy(bi).to(device), torch.from_numpy(tbi).to(device), 8)
    assert np.array_equal(got.cpu().numpy(), O.build_token_pair_mask(bi, tbi, 8))
    # a routed voxel geometry
    shape, chunk = (8, 8, 8), (4, 4, 4)
    idx = _distinct_indices(1, 2, 8, 8, 3, seed=1)
    tb = build_token_block_indices(shape, chunk, device=device)
    got = build_token_pair_mask(torch.from_numpy(idx).to(device), tb, 8).cpu().numpy()
    assert np.array_equal(got, O.build_token_pair_mask(idx, O.build_token_block_indices(shape, chunk), 8))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_block_major_permutation_exact(device, dtype):
    from lcv_bsa import reshape_from_block_major, reshape_to_block_major

    shape, chunk = (8, 12, 16), (4, 4, 4)
    x = _rand((1, 2, 8 * 12 * 16, 32), dtype, device, seed=2)
    bm = reshape_to_block_major(x, shape, chunk)
    assert np.array_equal(_np(bm), O.reshape_to_block_major(_np(x), shape, chunk))
    assert torch.equal(reshape_from_block_major(bm, shape, chunk), x)


# ---------------------------------------------------------------------------
# Launch order (scheduling): a permutation; results independent of it
# ---------------------------------------------------------------------------

def _attn_with_order(q, k, v, idx, shape, chunk, order, out=None):
    from lcv_bsa import _lib
    from lcv_bsa.block_sparse_attention import _geom, _strides

    B, H, S, D = q.shape
    out = torch.empty_like(q) if out is None else out
    st = _lib.load().lcv_bsa_attn_fwd(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), {torch.float16: 0, torch.bfloat16: 1,
                                                   torch.float32: 2}[q.dtype],
        B, H, S, D, _strides(q), _strides(k), _strides(v), idx.data_ptr(),
        order.data_ptr() if order is not None else None, idx.shape[3], 1.0 / math.sqrt(D),
        _geom(shape, chunk), out.data_ptr(), _strides(out), torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "attn")
    return out


@pytest.mark.parametrize("nb,k,heads", [(1, 1, 2), (7, 3, 2), (64, 4, 2), (900, 57, 2), (1024, 8, 2),
                                         (900, 57, 40), (1024, 8, 33), (1025, 8, 2), (4096, 5, 2)])
def test_schedule_permutation_sorted_by_key(device, nb, k, heads):
    """All three sorts: the rank sort with 64 keys per workgroup (nb <= 1024,
    at most 512 workgroups; 32-bit keys up to nb = 1023, 64-bit at 1024), the
    in-wave bitonic sort for larger grids (40 heads x 15 groups, 33 x 16) and
    the rank sort over several workgroups per head (1024 < nb <= 4096);
    padded entries count as nb."""
    from lcv_bsa import schedule_block_order

    idx = np.sort(_distinct_indices(1, heads, nb, nb, k, seed=nb + heads), axis=-1)
    if nb >= 7:
        idx[0, 0, 3, :] = -1  # padding sorts as nb
        idx[0, heads - 1, nb - 2, :] = -1
    order = schedule_block_order(torch.from_numpy(idx).to(device)).cpu().numpy()
    for h in range(heads):
        assert sorted(order[0, h].tolist()) == list(range(nb))
        first = np.where((idx[0, h, :, 0] >= 0), idx[0, h, :, 0], nb)
        med = np.where((idx[0, h, :, k // 2] >= 0), idx[0, h, :, k // 2], nb)
        keys = [(first[i], med[i], i) for i in order[0, h]]
        assert keys == sorted(keys)


@pytest.mark.parametrize("nq,nk,k", [(900, 1125, 71), (64, 300, 4), (1100, 2000, 9)])
def test_schedule_kv_sorts_by_kv_block_ids(device, nq, nk, k):
    """S_q != S_k routing: entries are K/V block ids up to nk > nq.  Lists
    that start at or above nq sort by their value (not as padding); only
    entries outside [0, nk) count as nk."""
    from lcv_bsa import schedule_block_order

    rng = np.random.default_rng(nq + nk)
    idx = np.sort(np.stack([rng.choice(nk, size=k, replace=False) for _ in range(2 * nq)]), axis=-1)
    idx = idx.reshape(1, 2, nq, k).astype(np.int32)
    idx[0, 1, 5, :] = -1
    idx[0, 1, 6, 0] = nk  # out of range: sorts as nk
    assert (idx[..., 0] >= nq).any()
    order = schedule_block_order(torch.from_numpy(idx).to(device), nk).cpu().numpy()
    for h in range(2):
        assert sorted(order[0, h].tolist()) == list(range(nq))
        first = np.where((idx[0, h, :, 0] >= 0) & (idx[0, h, :, 0] < nk), idx[0, h, :, 0], nk)
        med = np.where((idx[0, h, :, k // 2] >= 0) & (idx[0, h, :, k // 2] < nk), idx[0, h, :, k // 2], nk)
        keys = [(first[i], med[i], i) for i in order[0, h]]
        assert keys == sorted(keys)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_attention_launch_order_changes_only_rounding(device, dtype):
    from lcv_bsa import schedule_block_order

    shape, chunk = (1, 1, 4096), (1, 1, 64)
    D = 128 if dtype != torch.float32 else 64
    q, k, v = (_rand((1, 3, 4096, D), dtype, device, seed=s) for s in (21, 22, 23))
    idx = torch.from_numpy(np.sort(_distinct_indices(1, 3, 64, 64, 9, seed=5), axis=-1)).to(device)
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx.cpu().numpy(), shape, chunk)
    rnd = torch.stack([torch.randperm(64) for _ in range(3)])[None].to(torch.int32).to(device)
    outs = {}
    for name, order in (("identity", None), ("schedule", schedule_block_order(idx)), ("random", rnd)):
        outs[name] = _attn_with_order(q, k, v, idx, shape, chunk, order)
        assert_close_report(_np(outs[name]), ref, *TOL[dtype], f"attn order={name} {dtype}")
        # The same launch order always gives the same bits.
        assert torch.equal(outs[name], _attn_with_order(q, k, v, idx, shape, chunk, order))
    # The launch order sets where each q-block starts its (rotated) walk over
    # its tiles, which only changes the summation order: the orders agree to
    # a few output units in the last place.
    ulp = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7, torch.float32: 2.0 ** -23}[dtype]
    for name in ("schedule", "random"):
        d = (outs[name].float() - outs["identity"].float()).abs().max().item()
        assert d <= 4 * ulp, f"order={name}: max |diff| {d:.3g} > 4 ulp"


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_attention_launch_order_out_of_range_entries_launch_nothing(device, dtype):
    """A launch-order entry outside [0, nb) launches nothing: the q-block it
    would have named keeps what the output held, every other q-block is
    computed as usual (MFMA path for fp16, vector-ALU path for fp32)."""
    shape, chunk = (1, 1, 1024), (1, 1, 64)
    D = 128 if dtype != torch.float32 else 64
    q, k, v = (_rand((1, 2, 1024, D), dtype, device, seed=s) for s in (41, 42, 43))
    idx = torch.from_numpy(np.sort(_distinct_indices(1, 2, 16, 16, 4, seed=6), axis=-1)).to(device)
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx.cpu().numpy(), shape, chunk)
    order = torch.arange(16, dtype=torch.int32).repeat(1, 2, 1)
    order[0, 0, 3] = 16  # q-block 3 of head 0 is never launched
    order[0, 1, 5] = -7  # q-block 5 of head 1 is never launched
    out = torch.full_like(q, 7.0)
    _attn_with_order(q, k, v, idx, shape, chunk, order.to(device), out=out)
    expect = ref.copy()
    expect[0, 0, 3 * 64:4 * 64] = 7.0
    expect[0, 1, 5 * 64:6 * 64] = 7.0
    assert_close_report(_np(out), expect, *TOL[dtype], f"attn order with skipped entries {dtype}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("q_scale", [1.0, 6.0, 12.0])
def test_attn_wide_score_range_rescales(device, dtype, q_scale, D):
    """Scores that grow along each routing list (K block j scaled by 1 + j/4)
    and large q scales push later tiles far above the first tile's max, so
    the overflow guard acts: the workgroup walks the list again with the
    exact row maxima."""
    from lcv_bsa import bsa_attention_hip

    shape, chunk = (1, 1, 2048), (1, 1, 64)
    q, k, v, idx = wide_range_inputs(D, q_scale, dtype)
    out = bsa_attention_hip(q.to(device), k.to(device), v.to(device), torch.from_numpy(idx).to(device),
                            chunk, shape)
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx, shape, chunk)
    assert_close_report(_np(out), ref, *_wide_tol(dtype, D, q_scale), f"wide range q*{q_scale} {dtype} D={D}")


def _wide_tol(dtype, D, q_scale):
    """Tolerance of the wide-score-range tests.  With bf16 at D = 64 some
    outputs of these inputs reach |o| >= 4, where half a bf16 ulp is
    2^-6 = 1.6e-2: on the q-scale inputs the correctly rounded bf16 of the
    exact result already misses the fp64 oracle by 1.3-1.4e-2, above the
    general 1e-2.  Those
    cases get 2e-2 max-abs (pinned on the CPU by
    test_cpu_tolerance.py::test_bf16_wide_range_floor); the mean-abs bound and
    every other case keep the general tolerance."""
    max_abs, mean_abs = TOL[dtype]
    if dtype == torch.bfloat16 and D == 64:
        max_abs = 2e-2
    return max_abs, mean_abs


@pytest.mark.parametrize("D", [64, 128])
def test_attn_wide_range_long_lists(device, D):
    """The overflow guard with lists longer than one 64-entry chunk (top-k 96
    of 128 blocks, entries unsorted, one padding entry per row): the exact
    pass and the second walk both cross chunk boundaries."""
    from lcv_bsa import bsa_attention_hip

    S, nb, k = 8192, 128, 96
    shape, chunk = (1, 1, S), (1, 1, 64)
    q = _rand((1, 2, S, D), torch.float32, device, seed=51) * 8.0
    kk = _rand((1, 2, S, D), torch.float32, device, seed=52)
    kk = kk * (1.0 + torch.arange(S, device=device).div(64, rounding_mode="floor").float() / 16.0)[None, None, :, None]
    v = _rand((1, 2, S, D), torch.float32, device, seed=53)
    q, kk, v = q.half(), kk.half(), v.half()
    idx = _distinct_indices(1, 2, nb, nb, k, seed=54, sort=False)
    idx[:, :, :, 5] = -1  # padding: skipped
    out = bsa_attention_hip(q, kk, v, torch.from_numpy(idx).to(device), chunk, shape)
    ref = O.sparse_attention_from_indices(_np(q), _np(kk), _np(v), idx, shape, chunk)
    assert_close_report(_np(out), ref, *TOL[torch.float16], f"wide range, long lists, D={D}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("wide_rows", [(0, 32), (32, 64), (16, 48)])
def test_attn_wide_range_in_some_rows_only(device, dtype, wide_rows, D):
    """Only some query rows of each 64-row block see the growing scores (q
    scaled by 12 there), so in a workgroup one wave overflows its first-tile
    offset while the other does not (or both, for rows 16-48).
    Every row must still match the oracle, including the rows of a wave that
    had no overflow itself but walks again with its workgroup."""
    from lcv_bsa import bsa_attention_hip

    shape, chunk = (1, 1, 2048), (1, 1, 64)
    q, k, v, idx = wide_range_inputs(D, 12.0, dtype, seeds=(41, 42, 43), wide_rows=wide_rows)
    q, k, v = q.to(device), k.to(device), v.to(device)
    out = bsa_attention_hip(q, k, v, torch.from_numpy(idx).to(device), chunk, shape)
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx, shape, chunk)
    assert_close_report(_np(out), ref, *_wide_tol(dtype, D, 12.0), f"wide range in rows {wide_rows} {dtype} D={D}")
    out2 = bsa_attention_hip(q, k, v, torch.from_numpy(idx).to(device), chunk, shape)
    assert torch.equal(out, out2), "second run differs"


# ---------------------------------------------------------------------------
# S_q != S_k: queries over a longer (conditioning + noise) key sequence
# ---------------------------------------------------------------------------

KV_GEOMS = [
    ((4, 8, 8), (8, 8, 8), (4, 4, 4)),          # noise frames over cond + noise frames
    ((1, 1, 1024), (1, 1, 2560), (1, 1, 64)),   # contiguous 64-token blocks
    ((1, 1, 256), (1, 1, 64), (1, 1, 64)),      # fewer keys than queries
]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("geom", KV_GEOMS)
def test_attn_kv_matches_oracle(device, dtype, D, geom):
    from lcv_bsa import bsa_attention_hip

    q_shape, kv_shape, chunk = geom
    Sq, Sk = int(np.prod(q_shape)), int(np.prod(kv_shape))
    nq, nk = Sq // 64, Sk // 64
    q = _rand((2, 2, Sq, D), dtype, device, seed=21)
    k, v = (_rand((2, 2, Sk, D), dtype, device, seed=s) for s in (22, 23))
    for topk in sorted({1, min(3, nk), nk}):
        idx = _distinct_indices(2, 2, nq, nk, topk, seed=topk + D, sort=(topk != 3))
        out = bsa_attention_hip(q, k, v, torch.from_numpy(idx).to(device), chunk, q_shape, kv_shape=kv_shape)
        ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx, q_shape, chunk, kv_shape=kv_shape)
        assert out.shape == q.shape
        assert_close_report(_np(out), ref, *TOL[dtype], f"attn kv {dtype} D={D} {geom} k={topk}")


def test_attn_kv_padding_and_out_of_range(device):
    """Entries < 0 or >= nk are skipped; ids in [nq, nk) are real k-blocks."""
    from lcv_bsa import bsa_attention_hip

    q = _rand((1, 1, 128, 128), torch.float16, device, seed=31)
    k, v = (_rand((1, 1, 384, 128), torch.float16, device, seed=s) for s in (32, 33))
    idx = np.array([[[[5, -1, 4], [6, 2, -3]]]], dtype=np.int32)   # nk = 6: 6 and -3 are skipped
    out = bsa_attention_hip(q, k, v, torch.from_numpy(idx).to(device), (1, 1, 64), (1, 1, 128),
                            kv_shape=(1, 1, 384))
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), idx, (1, 1, 128), (1, 1, 64),
                                          kv_shape=(1, 1, 384))
    assert_close_report(_np(out), ref, *TOL[torch.float16], "kv padding")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_bsa_kv_end_to_end(device, dtype):
    """bsa_attention(..., kv_shape=): the noise half of a sequence attends to
    the whole of it.  Routing is the exact top-k of the pooled means' scores
    (the count rule over nk), and the output matches the oracle on it."""
    from lcv_bsa import bsa_attention
    from lcv_bsa.block_sparse_attention import mean_pool_blocks_3d

    full, noise, chunk = (8, 8, 16), (4, 8, 16), (4, 4, 4)
    S, Sq = int(np.prod(full)), int(np.prod(noise))
    q_all, k, v = (_rand((1, 2, S, 128), dtype, device, seed=s) for s in (41, 42, 43))
    q = q_all[:, :, S - Sq:]
    out, idx = bsa_attention(q, k, v, noise, sparsity=0.75, chunk_thw=chunk, return_indices=True,
                             kv_shape=full)
    nk = S // 64
    assert idx.shape[-1] == max(1, int(0.25 * nk))
    qb, kb = mean_pool_blocks_3d(q, noise, chunk), mean_pool_blocks_3d(k, full, chunk)
    ref_idx, _ = O.topk_block_indices(O.block_routing_scores(_np(qb), _np(kb)), top_k=idx.shape[-1])
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    ref = O.sparse_attention_from_indices(_np(q), _np(k), _np(v), ref_idx, noise, chunk, kv_shape=full)
    assert_close_report(_np(out), ref, *TOL[dtype], f"bsa kv {dtype}")
