"""CPU oracle: a NumPy restatement of the reference's Block Sparse Attention.

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` -- as the checker and the timed
CPU baseline, never by the product package.

Every function cites the reference lines it restates (paths relative to the
reference repository).  The reference runs on MLX (absent here), so this is a
restatement from its source, pinned by the reference's own known-answer and
invariant tests plus closed forms and brute force (tests/test_oracle.py).

Numerics: everything is evaluated in ``acc`` (float64 by default); fp16/bf16
inputs are first widened exactly.  ``topk_block_indices`` returns each row's
set sorted ascending, ties broken toward the lower block index.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import numpy as np

__all__ = [
    "mean_pool_blocks_3d", "block_routing_scores", "num_selected", "topk_block_indices",
    "build_token_block_indices", "build_token_pair_mask", "sdpa", "bsa_attention",
    "bsa_attention_masked", "sparse_attention_from_indices", "reshape_to_block_major",
    "reshape_from_block_major", "block_tokens", "rope_dims", "rope_freqs_3d", "rotate_half",
    "apply_rope", "executed_flops", "round_to", "rms_norm_fp32", "prepare_qk",
]


def _f(x, acc):
    return np.asarray(x).astype(acc, copy=False)


# --- block_sparse_attention.py:67-104 --------------------------------------
def mean_pool_blocks_3d(x, shape, chunk_thw=(4, 4, 4), acc=np.float64):
    """[B,H,S,D] -> [B,H,nb,D]: mean over each cT x cH x cW voxel, blocks in
    (bt, bh, bw) order.  Raises ValueError exactly where the reference does."""
    T, H_, W = shape
    cT, cH, cW = chunk_thw
    if T % cT or H_ % cH or W % cW:
        raise ValueError(
            f"Latent shape ({T}, {H_}, {W}) must be a multiple of chunk_thw {tuple(chunk_thw)}; "
            "refinement padding should guarantee this."
        )
    Bt, Bh, Bw = T // cT, H_ // cH, W // cW
    x = _f(x, acc)
    B, H, S, D = x.shape
    if S != T * H_ * W:
        raise ValueError(f"S={S} doesn't match T*H*W={T * H_ * W} for shape {tuple(shape)}")
    y = x.reshape(B, H, Bt, cT, Bh, cH, Bw, cW, D)
    y = y.transpose(0, 1, 2, 4, 6, 3, 5, 7, 8)
    y = y.reshape(B, H, Bt * Bh * Bw, cT * cH * cW, D)
    return y.mean(axis=3)


# --- block_sparse_attention.py:107-112 -------------------------------------
def block_routing_scores(q_blocks, k_blocks, acc=np.float64):
    """Unscaled q_blocks @ k_blocks^T."""
    return np.matmul(_f(q_blocks, acc), np.swapaxes(_f(k_blocks, acc), -1, -2))


# --- block_sparse_attention.py:127 ------------------------------------------
def num_selected(num_kv_blocks: int, sparsity: float) -> int:
    return max(1, int((1.0 - sparsity) * num_kv_blocks))


# --- block_sparse_attention.py:115-134 -------------------------------------
def topk_block_indices(score, sparsity: Optional[float] = None, top_k: Optional[int] = None):
    """Returns (indices [..., k] int32 ascending, k).  The reference takes the
    first k of argpartition(-score); the set is the same, its order there is
    unspecified.  Exact ties go to the lower index; NaN ranks last."""
    score = np.asarray(score)
    nk = score.shape[-1]
    k = num_selected(nk, sparsity) if top_k is None else int(top_k)
    if not 1 <= k <= nk:
        raise ValueError(f"top_k={k} must be in [1, {nk}]")
    neg = -score.astype(np.float64)
    nan = np.isnan(neg)
    neg[nan] = np.inf
    # primary key: NaN last; secondary: descending score; lexsort is stable,
    # so equal keys keep ascending index order.
    order = np.lexsort((neg, nan), axis=-1)[..., :k]
    return np.sort(order, axis=-1).astype(np.int32), k


# --- block_sparse_attention.py:137-159 -------------------------------------
def build_token_block_indices(shape, chunk_thw=(4, 4, 4)):
    T, H_, W = shape
    cT, cH, cW = chunk_thw
    Bh, Bw = H_ // cH, W // cW
    s = np.arange(T * H_ * W, dtype=np.int64)
    t = s // (H_ * W)
    hw = s % (H_ * W)
    h = hw // W
    w = hw % W
    return ((t // cT) * (Bh * Bw) + (h // cH) * Bw + (w // cW)).astype(np.int32)


# --- block_sparse_attention.py:162-198 -------------------------------------
def build_token_pair_mask(block_indices, token_block_index, num_kv_blocks: int):
    """[B,H,S,S] bool: True where block_of(s_k) is routed for block_of(s_q).

    Tokens whose block lies outside [0, nq) (query side) or [0, nk) (key
    side) get False; the reference's mx.take leaves such rows unspecified
    (its own test, test_bsa_tier_a_smoke.py:114-138, only asserts the
    in-range rows)."""
    bi = np.asarray(block_indices)
    B, H, nq, _ = bi.shape
    k_range = np.arange(num_kv_blocks)
    one_hot = bi[..., None] == k_range[None, None, None, None, :]
    block_pair = one_hot.any(axis=3)  # [B,H,nq,nk]
    tbi = np.asarray(token_block_index)
    S = tbi.shape[0]
    vq = (tbi >= 0) & (tbi < nq)
    vk = (tbi >= 0) & (tbi < num_kv_blocks)
    out = np.zeros((B, H, S, S), dtype=bool)
    rows = block_pair[:, :, tbi[vq]]                      # [B,H,Sq',nk]
    out[:, :, vq] = np.where(vk[None, None, None, :], rows[:, :, :, np.where(vk, tbi, 0)], False)
    return out


def sdpa(q, k, v, scale: float, mask=None, acc=np.float64):
    """Textbook softmax attention, softmax(scale*q k^T + mask) v (the
    semantics of mx.fast.scaled_dot_product_attention used at
    block_sparse_attention.py:248-250 and attention.py:179)."""
    q, k, v = _f(q, acc), _f(k, acc), _f(v, acc)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * acc(scale)
    if mask is not None:
        s = s + _f(mask, acc)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.matmul(p, v)


# --- block_sparse_attention.py:201-250 (literal Tier A form) ---------------
def bsa_attention_masked(q, k, v, shape, sparsity=0.9375, chunk_thw=(4, 4, 4),
                         sm_scale=None, top_k=None, acc=np.float64, return_indices=False):
    """Pool -> scores -> top-k -> [B,H,S,S] additive mask (0 / -1e9) -> SDPA.
    Memory is O(S^2): small inputs only."""
    q = np.asarray(q)
    D = q.shape[-1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    qb = mean_pool_blocks_3d(q, shape, chunk_thw)
    kb = mean_pool_blocks_3d(k, shape, chunk_thw)
    score = block_routing_scores(qb, kb)
    idx, _ = topk_block_indices(score, sparsity, top_k)
    tbi = build_token_block_indices(shape, chunk_thw)
    mask = build_token_pair_mask(idx, tbi, score.shape[-1])
    add = np.where(mask, 0.0, -1e9)
    out = sdpa(q, k, v, sm_scale, add, acc)
    return (out, idx) if return_indices else out


def block_tokens(shape, chunk_thw):
    """[nb, bs] t-major token of row r of block n (block-major row order,
    the layout _reshape_to_block_major produces, metal.py:185-205)."""
    T, H_, W = shape
    cT, cH, cW = chunk_thw
    Bh, Bw = H_ // cH, W // cW
    nb = (T // cT) * Bh * Bw
    n = np.arange(nb)
    bt, bh, bw = n // (Bh * Bw), (n // Bw) % Bh, n % Bw
    r = np.arange(cT * cH * cW)
    i, j, l = r // (cH * cW), (r // cW) % cH, r % cW
    return (bt * cT * H_ * W + bh * cH * W + bw * cW)[:, None] + (i * H_ * W + j * W + l)[None, :]


def sparse_attention_from_indices(q, k, v, block_indices, shape, chunk_thw=(4, 4, 4),
                                  sm_scale=None, acc=np.float64, q_blocks=None,
                                  heads: Optional[Sequence[tuple]] = None, kv_shape=None):
    """Attention of each q-block over the keys of its listed KV blocks -- the
    reference kernels' contract (block_sparse_attention_metal.py:75-164:
    entries listed twice count twice).  Entries outside [0, nk) are skipped.
    Equal to the masked Tier A form when the lists hold distinct valid blocks.

    ``kv_shape`` (default ``shape``) is the latent grid of k / v when their
    length differs from q's; the lists then hold k/v block ids.

    Returns [B,H,S,D] in ``acc`` (rows of q-blocks not computed are NaN when
    ``q_blocks`` restricts the set).  ``heads`` optionally restricts (b, h).
    """
    q, k, v = np.asarray(q), np.asarray(k), np.asarray(v)
    B, H, S, D = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    bt = block_tokens(shape, chunk_thw)
    btk = bt if kv_shape is None else block_tokens(kv_shape, chunk_thw)
    nb, bs = bt.shape
    nk = btk.shape[0]
    bi = np.asarray(block_indices)
    out = np.full((B, H, S, D), np.nan, dtype=acc)
    pairs = heads if heads is not None else [(b, h) for b in range(B) for h in range(H)]
    qsel = np.arange(nb) if q_blocks is None else np.asarray(q_blocks)
    for b, h in pairs:
        qh, kh, vh = _f(q[b, h], acc), _f(k[b, h], acc), _f(v[b, h], acc)
        for n in qsel:
            lst = bi[b, h, n]
            lst = lst[(lst >= 0) & (lst < nk)]
            tq = bt[n]
            if lst.size == 0:
                out[b, h, tq] = 0.0
                continue
            keys = btk[lst].reshape(-1)
            s = (qh[tq] @ kh[keys].T) * acc(sm_scale)
            s -= s.max(axis=-1, keepdims=True)
            p = np.exp(s)
            p /= p.sum(axis=-1, keepdims=True)
            out[b, h, tq] = p @ vh[keys]
    return out


def bsa_attention(q, k, v, shape, sparsity=0.9375, chunk_thw=(4, 4, 4), sm_scale=None,
                  top_k=None, acc=np.float64, return_indices=False, kv_shape=None):
    """Tier A result via the block-gathered form (no S^2 mask): equal to
    bsa_attention_masked because masked entries contribute exactly zero.

    ``kv_shape``: k / v over their own latent grid (S_k != S_q), pooled with
    the same voxel; the count rule then runs over the k-blocks.  The
    reference never routes this case through BSA (attention.py:89)."""
    qb = mean_pool_blocks_3d(q, shape, chunk_thw)
    kb = mean_pool_blocks_3d(k, shape if kv_shape is None else kv_shape, chunk_thw)
    idx, _ = topk_block_indices(block_routing_scores(qb, kb), sparsity, top_k)
    out = sparse_attention_from_indices(q, k, v, idx, shape, chunk_thw, sm_scale, acc, kv_shape=kv_shape)
    return (out, idx) if return_indices else out


# --- block_sparse_attention_metal.py:185-221 --------------------------------
def reshape_to_block_major(x, shape, chunk_thw):
    T, H_, W = shape
    cT, cH, cW = chunk_thw
    Bt, Bh, Bw = T // cT, H_ // cH, W // cW
    B, H, S, D = x.shape
    y = np.asarray(x).reshape(B, H, Bt, cT, Bh, cH, Bw, cW, D)
    return y.transpose(0, 1, 2, 4, 6, 3, 5, 7, 8).reshape(B, H, S, D)


def reshape_from_block_major(x, shape, chunk_thw):
    T, H_, W = shape
    cT, cH, cW = chunk_thw
    Bt, Bh, Bw = T // cT, H_ // cH, W // cW
    B, H, S, D = x.shape
    y = np.asarray(x).reshape(B, H, Bt, Bh, Bw, cT, cH, cW, D)
    return y.transpose(0, 1, 2, 5, 3, 6, 4, 7, 8).reshape(B, H, S, D)


# --- rope_3d.py:23-34, 53-128 ----------------------------------------------
def rope_dims(head_dim: int):
    return head_dim - 4 * (head_dim // 6), 2 * (head_dim // 6), 2 * (head_dim // 6)


def rope_freqs_3d(grid, head_dim: int, base: float = 10000.0):
    """[T*H*W, head_dim] angles (fp32 like the reference's precompute)."""
    T, H, W = grid
    dims = rope_dims(head_dim)
    parts = []
    for dim, n, ax in zip(dims, (T, H, W), range(3)):
        idx = np.arange(0, dim, 2, dtype=np.float32)[: dim // 2]
        inv = (1.0 / (np.float32(base) ** (idx / np.float32(dim)))).astype(np.float32)
        f = np.repeat(np.arange(n, dtype=np.float32)[:, None] * inv[None, :], 2, axis=-1)
        shp = [1, 1, 1, dim]
        shp[ax] = n
        parts.append(np.broadcast_to(f.reshape(shp), (T, H, W, dim)))
    return np.concatenate(parts, axis=-1).reshape(T * H * W, head_dim)


def rotate_half(x):
    x = np.asarray(x)
    x2 = x.reshape(*x.shape[:-1], x.shape[-1] // 2, 2)
    return np.stack([-x2[..., 1], x2[..., 0]], axis=-1).reshape(x.shape)


def apply_rope(x, freqs):
    xf = np.asarray(x).astype(np.float32)
    c, s = np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)
    return xf * c + rotate_half(xf) * s


# --- blocks.py:55-72 (RMSNorm_FP32), attention.py:191-201 -------------------
def round_to(x, dtype: str):
    """Round fp32 values to fp16 / bf16 (nearest even) and widen back to fp32."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        out = r.astype(np.uint32).view(np.float32)
        return np.where(np.isnan(x), x, out)
    return x


def rms_norm_fp32(x, weight=None, eps=1e-6, dtype="f16"):
    """RMSNorm_FP32 (blocks.py:55-72): x * rsqrt(mean(x^2) + eps) in fp32,
    rounded to the input dtype, then times the weight in that dtype."""
    x = np.asarray(x, dtype=np.float32)
    ms = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    y = round_to(x * (np.float32(1.0) / np.sqrt(ms + np.float32(eps))), dtype)
    if weight is None:
        return y
    return round_to(y * round_to(np.asarray(weight, dtype=np.float32), dtype), dtype)


def prepare_qk(q, k, grid, shape=None, chunk_thw=(4, 4, 4), q_weight=None, k_weight=None,
               eps=1e-6, dtype="f16"):
    """q_norm / k_norm then rope_3d (attention.py:195-201; RoPE in fp32 and
    rounded back, rope_3d.py:120-128), then the block means of the results
    (block_sparse_attention.py:67-104).  Returns q, k (dtype values as fp32)
    and their fp64 block means."""
    shape = tuple(grid) if shape is None else tuple(shape)
    f = rope_freqs_3d(grid, np.asarray(q).shape[-1]).astype(np.float32)
    cos, sin = np.cos(f), np.sin(f)
    outs = []
    for x, w in ((q, q_weight), (k, k_weight)):
        y = rms_norm_fp32(x, w, eps, dtype)
        r = round_to(y * cos + rotate_half(y) * sin, dtype)
        outs.append(r)
    means = [mean_pool_blocks_3d(o, shape, chunk_thw) for o in outs]
    return outs[0], outs[1], means[0], means[1]


def executed_flops(B, H, nq, k, D, bs=64):
    return 4 * B * H * nq * k * bs * bs * D
