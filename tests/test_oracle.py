"""Pins the CPU oracle before anything is compared against it.

Three kinds of checks, chosen so that a plausible mistake (dropped term,
wrong sign or index, transposed operand) fails at least one:

1. the reference's own known-answer / invariant tests for this path
   (tests/smoke/test_bsa_tier_a_smoke.py, test_bsa_tier_b_smoke.py,
   test_blocks_smoke.py:134-140), restated against the oracle;
2. independent computations: torch's CPU SDPA for dense attention,
   pure-Python brute force on tiny inputs, closed forms of RoPE;
3. planted mistakes: deliberately broken copies of oracle functions must be
   caught by the checks above (so the checks are not vacuous).
"""

from __future__ import annotations

import itertools
import math

import numpy as np
import pytest
import torch

from oracle import bsa_oracle as O

RNG = np.random.default_rng(1234)


def torch_sdpa(q, k, v, scale, mask=None):
    """Independent dense attention: torch CPU SDPA in fp64."""
    tq, tk, tv = (torch.from_numpy(np.asarray(x, dtype=np.float64)) for x in (q, k, v))
    am = None if mask is None else torch.from_numpy(np.asarray(mask, dtype=np.float64))
    return torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=am, scale=scale).numpy()


# ---------------------------------------------------------------------------
# 1. Reference known answers (test_bsa_tier_a_smoke.py)
# ---------------------------------------------------------------------------

def test_mean_pool_known_answer():
    """test_bsa_tier_a_smoke.py:47-65."""
    T, H_, W, D = 8, 8, 8, 4
    x = np.zeros((1, 2, T, H_, W, D), dtype=np.float32)
    x[:, :, :4, :4, :4, :] = 1.0
    y = O.mean_pool_blocks_3d(x.reshape(1, 2, T * H_ * W, D), (T, H_, W), (4, 4, 4))
    assert y.shape == (1, 2, 8, D)
    assert np.allclose(y[:, :, 0], 1.0)
    assert np.allclose(y[:, :, 1:], 0.0)


def test_routing_scores_known_answer():
    """test_bsa_tier_a_smoke.py:68-75: ones . twos over D=8 = 16."""
    s = O.block_routing_scores(np.ones((1, 1, 4, 8)), 2 * np.ones((1, 1, 4, 8)))
    assert s.shape == (1, 1, 4, 4)
    assert s[0, 0, 0, 0] == 16.0


def test_topk_count_rule():
    """test_bsa_tier_a_smoke.py:78-94: 0.75 of 8 keeps 2; the count clamps to 1."""
    idx, n = O.topk_block_indices(RNG.normal(size=(1, 2, 4, 8)), sparsity=0.75)
    assert idx.shape == (1, 2, 4, 2) and n == 2
    assert (idx >= 0).all() and (idx < 8).all()
    _, n1 = O.topk_block_indices(RNG.normal(size=(1, 1, 2, 4)), sparsity=0.99)
    assert n1 == 1
    # the rule is a floor: 0.0625 * 900 = 56.25 -> 56, 450 -> 28
    assert O.num_selected(900, 0.9375) == 56 and O.num_selected(450, 0.9375) == 28


def test_token_block_indices_known_answer():
    """test_bsa_tier_a_smoke.py:97-111."""
    assert (O.build_token_block_indices((4, 4, 4), (4, 4, 4)) == 0).all()
    t2 = O.build_token_block_indices((8, 4, 4), (4, 4, 4))
    assert t2.shape == (128,) and (t2[:64] == 0).all() and (t2[64:] == 1).all()


def test_token_pair_mask_known_answer():
    """test_bsa_tier_a_smoke.py:114-138."""
    bi = np.array([[[[3, 5], [0, 7]]]], dtype=np.int32)
    m = O.build_token_pair_mask(bi, np.arange(8, dtype=np.int32), 8)
    assert m.shape == (1, 1, 8, 8)
    assert m[0, 0, 0, 3] and m[0, 0, 0, 5] and not m[0, 0, 0, 0]
    assert m[0, 0, 1, 0] and m[0, 0, 1, 7] and not m[0, 0, 1, 3]


def test_sparsity_zero_equals_dense():
    """test_bsa_tier_a_smoke.py:141-162: sparsity=0 == dense SDPA, < 1e-4 in fp32."""
    q, k, v = (RNG.normal(size=(1, 4, 64, 16)).astype(np.float32) for _ in range(3))
    out = O.bsa_attention_masked(q, k, v, (4, 4, 4), sparsity=0.0, acc=np.float32)
    dense = torch_sdpa(q, k, v, 1.0 / math.sqrt(16))
    assert np.abs(out - dense).max() < 1e-4
    out_g = O.bsa_attention(q, k, v, (4, 4, 4), sparsity=0.0)
    assert np.abs(out_g - dense).max() < 1e-10


def test_realistic_shape_finite():
    """test_bsa_tier_a_smoke.py:165-184."""
    T, H_, W, D = 4, 8, 8, 32
    q, k, v = (RNG.normal(size=(1, 2, T * H_ * W, D)) for _ in range(3))
    out = O.bsa_attention_masked(q, k, v, (T, H_, W), sparsity=0.9375)
    assert out.shape == (1, 2, T * H_ * W, D) and np.isfinite(out).all()


def test_rejects_non_multiple_shape():
    """test_bsa_tier_a_smoke.py:187-196."""
    q = np.zeros((1, 1, 96, 8))
    with pytest.raises(ValueError, match="multiple of"):
        O.bsa_attention_masked(q, q, q, (4, 4, 6), sparsity=0.9)
    with pytest.raises(ValueError, match="doesn't match"):
        O.mean_pool_blocks_3d(np.zeros((1, 1, 100, 8)), (4, 4, 4))


def test_rotate_half_known_answer():
    """test_blocks_smoke.py:134-140."""
    assert O.rotate_half(np.array([[1.0, 2.0, 3.0, 4.0]])).tolist() == [[-2.0, 1.0, -4.0, 3.0]]


# ---------------------------------------------------------------------------
# 1b. Kernel gates of test_bsa_tier_b_smoke.py, on the gathered form
# ---------------------------------------------------------------------------

def test_gathered_single_block_equals_dense():
    """test_bsa_tier_b_smoke.py:47-79: one q-block, one KV block == dense."""
    q, k, v = (RNG.normal(size=(1, 2, 64, 16)) for _ in range(3))
    out = O.sparse_attention_from_indices(q, k, v, np.zeros((1, 2, 1, 1), np.int32), (4, 4, 4))
    assert np.abs(out - torch_sdpa(q, k, v, 0.25)).max() < 1e-12


def test_gathered_arange_equals_tier_a_dense():
    """test_bsa_tier_b_smoke.py:82-117: all blocks listed == Tier A sparsity 0."""
    q, k, v = (RNG.normal(size=(1, 2, 128, 16)) for _ in range(3))
    bi = np.broadcast_to(np.arange(2, dtype=np.int32), (1, 2, 2, 2))
    out = O.sparse_attention_from_indices(q, k, v, bi, (8, 4, 4))
    ref = O.bsa_attention_masked(q, k, v, (8, 4, 4), sparsity=0.0)
    assert np.abs(out - ref).max() < 1e-12


@pytest.mark.parametrize("shape,chunk,sparsity", [
    ((8, 8, 8), (4, 4, 4), 0.5),
    ((8, 12, 16), (4, 4, 4), 0.75),
    ((1, 1, 512), (1, 1, 64), 0.75),
    ((4, 8, 8), (2, 2, 2), 0.9),
])
def test_gathered_equals_masked_same_routing(shape, chunk, sparsity):
    """test_bsa_tier_b_smoke.py:120-160, on several geometries."""
    S = int(np.prod(shape))
    q, k, v = (RNG.normal(size=(1, 3, S, 16)) for _ in range(3))
    out_m, idx = O.bsa_attention_masked(q, k, v, shape, sparsity, chunk, return_indices=True)
    out_g = O.sparse_attention_from_indices(q, k, v, idx, shape, chunk)
    assert np.abs(out_g - out_m).max() < 1e-12


# ---------------------------------------------------------------------------
# 2. Brute force and closed forms
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape,chunk", [((8, 12, 16), (4, 4, 4)), ((4, 6, 8), (2, 3, 4)),
                                         ((1, 1, 256), (1, 1, 64)), ((4, 4, 4), (1, 2, 4))])
def test_pool_brute_force(shape, chunk):
    T, H_, W = shape
    cT, cH, cW = chunk
    x = RNG.normal(size=(2, 2, T * H_ * W, 3))
    y = O.mean_pool_blocks_3d(x, shape, chunk)
    tbi = O.build_token_block_indices(shape, chunk)
    nb = y.shape[2]
    for b, h in itertools.product(range(2), range(2)):
        for n in range(nb):
            toks = [s for s in range(T * H_ * W) if tbi[s] == n]
            assert len(toks) == cT * cH * cW
            assert np.allclose(y[b, h, n], x[b, h, toks].mean(axis=0), atol=1e-14)


def test_token_block_brute_force():
    shape, chunk = (6, 8, 12), (2, 4, 3)
    T, H_, W = shape
    tbi = O.build_token_block_indices(shape, chunk)
    Bh, Bw = H_ // chunk[1], W // chunk[2]
    for s in range(T * H_ * W):
        t, rem = divmod(s, H_ * W)
        h, w = divmod(rem, W)
        assert tbi[s] == (t // chunk[0]) * Bh * Bw + (h // chunk[1]) * Bw + w // chunk[2]


def test_block_tokens_inverts_token_blocks():
    shape, chunk = (8, 12, 16), (4, 4, 4)
    bt = O.block_tokens(shape, chunk)
    tbi = O.build_token_block_indices(shape, chunk)
    assert sorted(bt.reshape(-1).tolist()) == list(range(int(np.prod(shape))))
    for n in range(bt.shape[0]):
        assert (tbi[bt[n]] == n).all()


def test_topk_brute_force_with_ties_and_nan():
    for trial in range(40):
        nk = int(RNG.integers(1, 40))
        k = int(RNG.integers(1, nk + 1))
        sc = RNG.integers(-3, 4, size=(2, 3, nk)).astype(np.float64)  # many exact ties
        if trial % 4 == 0:
            sc[RNG.random(sc.shape) < 0.2] = np.nan
        if trial % 3 == 0:
            sc[RNG.random(sc.shape) < 0.2] = -np.inf
        if trial % 5 == 0:
            sc[sc == 0] = -0.0
        idx, kk = O.topk_block_indices(sc, top_k=k)
        assert kk == k
        for b, h in itertools.product(range(2), range(3)):
            row = sc[b, h]
            key = lambda j: (1, 0.0, j) if math.isnan(row[j]) else (0, -row[j], j)
            expect = sorted(sorted(range(nk), key=key)[:k])
            assert idx[b, h].tolist() == expect


def test_masked_attention_brute_force():
    """The masked Tier A path against explicit per-query Python loops."""
    shape, chunk = (2, 4, 16), (1, 2, 16)   # 128 tokens, 4 voxel blocks of 32
    S, D = 128, 5
    q, k, v = (RNG.normal(size=(1, 1, S, D)) for _ in range(3))
    out, idx = O.bsa_attention_masked(q, k, v, shape, sparsity=0.5, chunk_thw=chunk,
                                      return_indices=True)
    tbi = O.build_token_block_indices(shape, chunk)
    scale = 1.0 / math.sqrt(D)
    for sq in range(S):
        allowed = [sk for sk in range(S) if tbi[sk] in set(idx[0, 0, tbi[sq]].tolist())]
        s = [scale * sum(q[0, 0, sq, d] * k[0, 0, sk, d] for d in range(D)) for sk in allowed]
        m = max(s)
        w = [math.exp(x - m) for x in s]
        z = sum(w)
        expect = [sum(w[i] * v[0, 0, sk, d] for i, sk in enumerate(allowed)) / z for d in range(D)]
        assert np.allclose(out[0, 0, sq], expect, atol=1e-12)


def test_duplicates_and_padding_semantics():
    """Listed-twice blocks count twice (the reference kernels' loop); -1 skips."""
    q, k, v = (RNG.normal(size=(1, 1, 128, 8)) for _ in range(3))
    shape, chunk = (1, 1, 128), (1, 1, 64)
    a = O.sparse_attention_from_indices(q, k, v, np.array([[[[0, -1], [1, 5]]]]), shape, chunk)
    b = O.sparse_attention_from_indices(q, k, v, np.array([[[[0, 0], [1, 1]]]]), shape, chunk)
    c = O.sparse_attention_from_indices(q, k, v, np.array([[[[0], [1]]]]), shape, chunk)
    assert np.abs(a - c).max() < 1e-13 and np.abs(b - c).max() < 1e-13  # weights renormalise
    z = O.sparse_attention_from_indices(q, k, v, np.array([[[[-1], [-1]]]]), shape, chunk)
    assert (z == 0).all()


def test_block_major_roundtrip():
    x = RNG.normal(size=(1, 2, 8 * 12 * 16, 3))
    shape, chunk = (8, 12, 16), (4, 4, 4)
    bm = O.reshape_to_block_major(x, shape, chunk)
    assert np.array_equal(O.reshape_from_block_major(bm, shape, chunk), x)
    bt = O.block_tokens(shape, chunk)
    assert np.array_equal(bm.reshape(1, 2, -1, 64, 3), x[:, :, bt])
    y = RNG.normal(size=(1, 1, 256, 2))
    assert np.array_equal(O.reshape_to_block_major(y, (1, 1, 256), (1, 1, 64)), y)


def test_rope_closed_forms():
    assert O.rope_dims(128) == (44, 42, 42)
    grid, D = (3, 4, 5), 128
    f = O.rope_freqs_3d(grid, D)
    assert f.shape == (60, D)
    assert (f[0] == 0).all()  # position (0,0,0): identity rotation
    x = RNG.normal(size=(1, 1, 60, D)).astype(np.float32)
    y = O.apply_rope(x, f)
    assert np.allclose(y[0, 0, 0], x[0, 0, 0])
    # each adjacent pair is rotated: pair norms are preserved
    n_x = (x.reshape(60, D // 2, 2) ** 2).sum(-1)
    n_y = (y.reshape(60, D // 2, 2) ** 2).sum(-1)
    assert np.allclose(n_x, n_y, rtol=1e-5)
    # t-part of token (t, h, w) uses angle t * 10000^(-2i/44) on pair i
    t, h, w = 2, 3, 1
    s = t * 20 + h * 5 + w
    i = 3
    assert np.isclose(f[s, 2 * i], t * 10000.0 ** (-2 * i / 44), rtol=1e-6)
    assert f[s, 2 * i] == f[s, 2 * i + 1]
    assert np.isclose(f[s, 44 + 2 * i], h * 10000.0 ** (-2 * i / 42), rtol=1e-6)
    assert np.isclose(f[s, 86 + 2 * i], w * 10000.0 ** (-2 * i / 42), rtol=1e-6)


def test_rope_relative_position():
    """<R(p) a, R(p') b> depends only on p - p' (a rotation property)."""
    D = 24
    grid = (6, 6, 6)
    f = O.rope_freqs_3d(grid, D).astype(np.float64)
    a = RNG.normal(size=D)
    b = RNG.normal(size=D)

    def rot(x, s):
        return x * np.cos(f[s]) + O.rotate_half(x) * np.sin(f[s])

    def tok(t, h, w):
        return (t * 6 + h) * 6 + w

    d1 = rot(a, tok(3, 2, 4)) @ rot(b, tok(1, 1, 1))
    d2 = rot(a, tok(4, 3, 5)) @ rot(b, tok(2, 2, 2))
    assert abs(d1 - d2) < 1e-4


# ---------------------------------------------------------------------------
# 3. Planted mistakes must be caught
# ---------------------------------------------------------------------------

def test_planted_transposed_key_is_caught():
    def bad_sdpa(q, k, v, scale):
        s = np.matmul(k, q.swapaxes(-1, -2)) * scale  # transposed scores
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        return np.matmul(p / p.sum(-1, keepdims=True), v)

    q, k, v = (RNG.normal(size=(1, 2, 64, 16)) for _ in range(3))
    assert np.abs(bad_sdpa(q, k, v, 0.25) - torch_sdpa(q, k, v, 0.25)).max() > 1e-3
    assert np.abs(O.sdpa(q, k, v, 0.25) - torch_sdpa(q, k, v, 0.25)).max() < 1e-12


def test_planted_bottom_k_is_caught():
    sc = RNG.normal(size=(1, 1, 3, 16))
    good, _ = O.topk_block_indices(sc, top_k=4)
    bad = np.sort(np.argsort(sc, axis=-1)[..., :4], axis=-1)  # sign error: bottom-k
    brute = np.array([[[sorted(np.argsort(-r)[:4]) for r in sc[0, 0]]]])
    assert np.array_equal(good, brute) and not np.array_equal(bad, brute)


def test_planted_missing_voxel_transpose_is_caught():
    T, H_, W, D = 8, 8, 8, 1
    x = np.zeros((1, 1, T, H_, W, D))
    x[:, :, 4:, :4, :4] = 1.0  # block (bt=1, bh=0, bw=0) = flat index 4
    flat = x.reshape(1, 1, -1, D)
    good = O.mean_pool_blocks_3d(flat, (T, H_, W), (4, 4, 4))
    bad = flat.reshape(1, 1, 8, 64, D).mean(axis=3)  # contiguous runs, no voxel transpose
    assert good[0, 0, 4, 0] == 1.0 and np.count_nonzero(good) == 1
    assert not np.array_equal(bad, good)


def test_planted_floor_vs_ceil_is_caught():
    ceil_rule = lambda nk, sp: max(1, math.ceil((1.0 - sp) * nk))
    assert ceil_rule(900, 0.9375) != O.num_selected(900, 0.9375)


# ---------------------------------------------------------------------------
# RMSNorm_FP32 and dtype rounding (blocks.py:55-72; attention.py:195-201)
# ---------------------------------------------------------------------------

def test_round_to_matches_torch_and_ties_to_even():
    x = RNG.normal(size=4096).astype(np.float32) * np.float32(100.0)
    for name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        ref = torch.from_numpy(x).to(dt).float().numpy()
        assert np.array_equal(O.round_to(x, name), ref), name
    one = np.float32(1.0)
    assert O.round_to(one + np.float32(2.0 ** -11), "f16") == 1.0           # tie -> even
    assert O.round_to(one + np.float32(3 * 2.0 ** -11), "f16") == one + np.float32(2.0 ** -9)
    assert O.round_to(one + np.float32(2.0 ** -8), "bf16") == 1.0           # tie -> even
    assert O.round_to(one + np.float32(3 * 2.0 ** -8), "bf16") == one + np.float32(2.0 ** -6)
    assert np.isnan(O.round_to(np.float32(np.nan), "bf16"))
    assert O.round_to(np.float32(np.inf), "bf16") == np.inf


def test_rms_norm_known_answers():
    # [3, 4]: mean(x^2) = 12.5, so x / sqrt(12.5) (eps 0 here).
    got = O.rms_norm_fp32(np.array([[3.0, 4.0]]), eps=0.0, dtype="f32")
    assert np.allclose(got, np.array([[3.0, 4.0]]) / math.sqrt(12.5), rtol=1e-6)
    # a constant row normalises to +-1 (up to eps); the weight scales per column.
    c = np.full((2, 8), -7.0, np.float32)
    assert np.allclose(O.rms_norm_fp32(c, eps=1e-6, dtype="f32"), -1.0, atol=1e-6)
    w = np.arange(1, 9, dtype=np.float32)
    assert np.allclose(O.rms_norm_fp32(c, w, eps=1e-6, dtype="f32"), -w, rtol=1e-6)
    # fp16 / bf16: fp64 truth rounded to the dtype (normalisation) and again
    # after the weight; one dtype ulp at most from the double-precision value.
    x = RNG.normal(size=(64, 128)).astype(np.float32)
    wt = (1.0 + 0.1 * RNG.normal(size=128)).astype(np.float32)
    for name, ulp in (("f16", 2.0 ** -10), ("bf16", 2.0 ** -7)):
        wq = O.round_to(wt, name)
        x64 = x.astype(np.float64)
        truth = x64 / np.sqrt(np.mean(x64 * x64, axis=-1, keepdims=True) + 1e-6) * wq
        got = O.rms_norm_fp32(x, wt, 1e-6, name)
        assert np.all(np.abs(got - truth) <= 2 * ulp * np.maximum(np.abs(truth), 1.0)), name


def test_planted_rms_sum_instead_of_mean_is_caught():
    x = RNG.normal(size=(4, 128)).astype(np.float32)
    planted = x / np.sqrt(np.sum(x * x, axis=-1, keepdims=True) + 1e-6)
    assert not np.allclose(planted, O.rms_norm_fp32(x, eps=1e-6, dtype="f32"), rtol=1e-3)


def test_prepare_qk_composes_the_pinned_steps():
    """prepare_qk == rms_norm -> RoPE (fp32, rounded) -> block means; with a
    one-position grid RoPE is the identity."""
    q = RNG.normal(size=(1, 2, 64, 64)).astype(np.float32)
    k = RNG.normal(size=(1, 2, 64, 64)).astype(np.float32)
    qo, ko, qb, kb = O.prepare_qk(q, k, (1, 1, 64), chunk_thw=(1, 1, 64), dtype="f16")
    r = O.rms_norm_fp32(q, None, 1e-6, "f16")
    f = O.rope_freqs_3d((1, 1, 64), 64).astype(np.float32)
    assert np.array_equal(qo, O.round_to(r * np.cos(f) + O.rotate_half(r) * np.sin(f), "f16"))
    assert np.allclose(qb, O.mean_pool_blocks_3d(qo, (1, 1, 64), (1, 1, 64)))
    # Position 0 on every axis: cos = 1, sin = 0.
    q1 = RNG.normal(size=(1, 1, 64, 64)).astype(np.float32)
    qo1, _, _, _ = O.prepare_qk(q1, q1, (64, 1, 1), shape=(1, 1, 64), chunk_thw=(1, 1, 64))
    f1 = O.rope_freqs_3d((64, 1, 1), 64)
    assert np.all(f1[0] == 0.0)
    assert np.array_equal(qo1[..., 0, :], O.rms_norm_fp32(q1, None, 1e-6, "f16")[..., 0, :])


# ---------------------------------------------------------------------------
# S_q != S_k (queries over a longer key sequence)
# ---------------------------------------------------------------------------

def test_kv_shape_all_blocks_is_dense_over_all_keys():
    """Noise queries (the last frames) over conditioning + noise keys: with
    every k-block selected the gathered form is dense attention of q over
    all of k (torch's SDPA), for voxel and contiguous geometries."""
    rng = np.random.default_rng(5)
    for q_shape, kv_shape, chunk in (((4, 8, 8), (8, 8, 8), (4, 4, 4)),
                                     ((1, 1, 256), (1, 1, 448), (1, 1, 64))):
        Sq, Sk = int(np.prod(q_shape)), int(np.prod(kv_shape))
        q = rng.normal(size=(1, 2, Sq, 16))
        k = rng.normal(size=(1, 2, Sk, 16))
        v = rng.normal(size=(1, 2, Sk, 16))
        nk = Sk // 64
        out, idx = O.bsa_attention(q, k, v, q_shape, chunk_thw=chunk, top_k=nk, return_indices=True,
                                   kv_shape=kv_shape)
        assert idx.shape == (1, 2, Sq // 64, nk)
        assert np.allclose(out, torch_sdpa(q, k, v, 0.25), atol=1e-12)


def test_kv_shape_equal_grids_match_square_form():
    rng = np.random.default_rng(6)
    shape = (4, 8, 8)
    q, k, v = (rng.normal(size=(1, 2, 256, 16)) for _ in range(3))
    a = O.bsa_attention(q, k, v, shape, top_k=2)
    b = O.bsa_attention(q, k, v, shape, top_k=2, kv_shape=shape)
    assert np.array_equal(a, b)


def test_kv_shape_routes_over_key_blocks():
    """Each q-block keeps the top-k k-blocks of the longer key grid: plant a
    key block that matches q-block 0 exactly and check it is selected, and
    that k-block ids beyond nq occur (the lists index k, not q)."""
    rng = np.random.default_rng(7)
    Sq, Sk = 128, 320
    q = rng.normal(size=(1, 1, Sq, 16)) * 0.1
    k = rng.normal(size=(1, 1, Sk, 16)) * 0.1
    v = rng.normal(size=(1, 1, Sk, 16))
    direction = np.zeros(16)
    direction[3] = 5.0
    q[0, 0, :64] += direction
    k[0, 0, 256:320] += direction            # k-block 4 (beyond nq = 2)
    _, idx = O.bsa_attention(q, k, v, (1, 1, Sq), chunk_thw=(1, 1, 64), top_k=1, return_indices=True,
                             kv_shape=(1, 1, Sk))
    assert idx[0, 0, 0, 0] == 4
