"""CPU oracle: a NumPy restatement of one LongCat-Video DiT block.

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/`` as the checker of the
torch + HIP block (``lcv_bsa.dit_block``), never by the product package.

Restates ``LongCatSingleStreamBlock.__call__`` (longcat_video/models/
longcat_video_dit.py:80-138) with its parts: ``LayerNorm_FP32`` and
``modulate_fp32`` (blocks.py:79-119), ``RMSNorm_FP32`` (blocks.py:55-72, in
bsa_oracle), ``FeedForwardSwiGLU`` (blocks.py:23-51), the self-attention
layer (attention.py:186-233, with the conditioning split of 202-221) with
BSA through bsa_oracle, and ``MultiHeadCrossAttention`` (attention.py:
282-371, one batch item, so the block-diagonal text mask is all zeros).

Numerics follow the reference's dtypes: tensors between modules hold the
model dtype (``round_to`` after every op that produces one), the AdaLN
parameters, modulation and gated residuals are fp32.  Matrix products are
evaluated in fp64 and rounded once, standing for an fp32-accumulating GEMM.
Parameters use the PyTorch checkpoint's key names.
"""

from __future__ import annotations

from typing import Optional, Sequence

import numpy as np

from . import bsa_oracle as B

__all__ = [
    "silu", "swiglu_hidden_dim", "layer_norm_fp32", "modulate_fp32", "linear", "feed_forward_swiglu",
    "dense_attention", "self_attention", "self_attention_kv_cache", "cross_attention", "dit_block",
    "block_param_shapes",
]

F32 = np.float32


def _r(x, dtype):
    return B.round_to(np.asarray(x, dtype=np.float64).astype(F32), dtype) if dtype != "f32" else np.asarray(x, F32)


def silu(x):
    """x * sigmoid(x) (mlx.nn.silu), evaluated in fp64."""
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def swiglu_hidden_dim(hidden_dim: int, multiple_of: int = 256, ffn_dim_multiplier: Optional[float] = None) -> int:
    """The inner width of FeedForwardSwiGLU (blocks.py:37-44): 2/3 rule, then
    rounded up to ``multiple_of``."""
    h = int(2 * hidden_dim / 3)
    if ffn_dim_multiplier is not None:
        h = int(ffn_dim_multiplier * h)
    return multiple_of * ((h + multiple_of - 1) // multiple_of)


def layer_norm_fp32(x, weight=None, bias=None, eps: float = 1e-6):
    """LayerNorm_FP32 (blocks.py:79-103) on fp32 values: population variance,
    (x - mean) * rsqrt(var + eps), then the optional affine; returns fp32."""
    x = np.asarray(x, np.float64)
    mean = x.mean(-1, keepdims=True)
    var = ((x - mean) ** 2).mean(-1, keepdims=True)
    y = (x - mean) / np.sqrt(var + eps)
    if weight is not None:
        y = y * np.asarray(weight, np.float64) + np.asarray(bias, np.float64)
    return y.astype(F32)


def modulate_fp32(x, shift, scale, dtype: str, eps: float = 1e-6):
    """modulate_fp32 with a no-affine LayerNorm_FP32 (blocks.py:106-119):
    ``LN(x) * (scale + 1) + shift`` in fp32, cast to the model dtype.  ``x``
    is [B, T, n, C]; ``shift`` / ``scale`` broadcast as [B, T, 1, C]."""
    y = layer_norm_fp32(x, eps=eps).astype(np.float64)
    y = y * (np.asarray(scale, np.float64) + 1.0) + np.asarray(shift, np.float64)
    return _r(y, dtype)


def linear(x, w, b=None, dtype: str = "bf16"):
    """nn.Linear in the model dtype: x @ w.T (+ b), accumulated wide, rounded once."""
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    if b is not None:
        y = y + np.asarray(b, np.float64)
    return _r(y, dtype)


def feed_forward_swiglu(x, w1, w2, w3, dtype: str):
    """FeedForwardSwiGLU.__call__ (blocks.py:50-51): w2(silu(w1 x) * w3 x),
    each intermediate held in the model dtype."""
    a = _r(silu(linear(x, w1, dtype=dtype)), dtype)
    g = _r(a.astype(np.float64) * linear(x, w3, dtype=dtype), dtype)
    return linear(g, w2, dtype=dtype)


def dense_attention(q, k, v, scale: float):
    """softmax(q k^T * scale) v over the last two axes, fp64."""
    q, k, v = (np.asarray(a, np.float64) for a in (q, k, v))
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    return (p / p.sum(-1, keepdims=True)) @ v


def _branch(q, k, v, geom, kv_geom, top_k, idx):
    """One attention call of the layer: BSA over ``geom`` = (shape, chunk)
    (k / v over ``kv_geom`` when they are longer; routing ``idx`` if given,
    else the top-k of the pooled means), or dense attention when ``geom`` is
    None.  Returns (out, idx)."""
    D = q.shape[-1]
    if geom is None:
        return dense_attention(q, k, v, D ** -0.5), None
    shape, chunk = geom
    kv_shape = None if kv_geom is None else kv_geom[0]
    if idx is None:
        qb = B.mean_pool_blocks_3d(q, shape, chunk)
        kb = B.mean_pool_blocks_3d(k, shape if kv_shape is None else kv_shape, chunk)
        idx, _ = B.topk_block_indices(B.block_routing_scores(qb, kb), top_k=top_k)
    return B.sparse_attention_from_indices(q, k, v, idx, shape, chunk, D ** -0.5, kv_shape=kv_shape), idx


def self_attention(x, p, latent_shape, num_heads: int, dtype: str, bsa: dict, block_indices=None,
                   num_cond_latents: int = 0):
    """Attention.__call__ (attention.py:186-233): fused QKV, q_norm / k_norm,
    rope_3d over the latent grid, then either one attention over all tokens
    (``bsa["all"]``) or, with conditioning latents, the split of attention.py:
    202-221: the conditioning tokens among themselves (``bsa["cond"]``) and
    the noise queries over all keys (``bsa["noise"]`` = (q geometry, k/v
    geometry), dense in the reference).  Each ``bsa`` entry is a
    (shape, chunk) geometry or None for dense; ``bsa["top_k"]`` is the count.
    ``block_indices`` maps branch name -> routing to use.  Returns (out,
    {branch: routing})."""
    Bsz, N, C = x.shape
    H, D = num_heads, C // num_heads
    qkv = linear(x, p["attn.qkv.weight"], p["attn.qkv.bias"], dtype).reshape(Bsz, N, 3, H, D)
    q, k, v = (np.transpose(qkv[:, :, i], (0, 2, 1, 3)) for i in range(3))
    q = B.rms_norm_fp32(q, p["attn.q_norm.weight"], 1e-6, dtype)
    k = B.rms_norm_fp32(k, p["attn.k_norm.weight"], 1e-6, dtype)
    f = B.rope_freqs_3d(tuple(latent_shape), D).astype(F32)
    cos, sin = np.cos(f), np.sin(f)
    q = B.round_to(q * cos + B.rotate_half(q) * sin, dtype)
    k = B.round_to(k * cos + B.rotate_half(k) * sin, dtype)
    given = block_indices or {}
    idx = {}
    if num_cond_latents:
        nc = N // latent_shape[0] * num_cond_latents
        oc, idx["cond"] = _branch(q[:, :, :nc], k[:, :, :nc], v[:, :, :nc], bsa.get("cond"), None,
                                  bsa["top_k"], given.get("cond"))
        gq, gk = bsa.get("noise") or (None, None)
        on, idx["noise"] = _branch(q[:, :, nc:], k, v, gq, gk, bsa["top_k"], given.get("noise"))
        o = np.concatenate([oc, on], axis=2)
    else:
        o, idx["all"] = _branch(q, k, v, bsa.get("all"), None, bsa["top_k"], given.get("all"))
    o = _r(o, dtype)
    o = np.transpose(o, (0, 2, 1, 3)).reshape(Bsz, N, C)
    return linear(o, p["attn.proj.weight"], p["attn.proj.bias"], dtype), idx


def self_attention_kv_cache(x, p, latent_shape, num_heads: int, dtype: str, kv_cache, num_cond_latents: int,
                            bsa: dict, block_indices=None):
    """Attention.forward_with_kv_cache (attention.py:235-275): fresh q / k / v
    of the current chunk, k / v appended to the cache (normed, not rotated);
    with conditioning latents RoPE runs over the extended grid with q
    zero-padded at the cache positions; then the queries attend to all keys
    (``bsa["noise"]`` geometry pair, or None = dense as in the reference).
    Returns (out, {"noise": routing})."""
    Bsz, N, C = x.shape
    H, D = num_heads, C // num_heads
    qkv = linear(x, p["attn.qkv.weight"], p["attn.qkv.bias"], dtype).reshape(Bsz, N, 3, H, D)
    q, k, v = (np.transpose(qkv[:, :, i], (0, 2, 1, 3)) for i in range(3))
    q = B.rms_norm_fp32(q, p["attn.q_norm.weight"], 1e-6, dtype)
    k = B.rms_norm_fp32(k, p["attn.k_norm.weight"], 1e-6, dtype)
    k_cache, v_cache = (np.asarray(a, F32) for a in kv_cache)
    k_full = np.concatenate([k_cache, k], axis=2)
    v_full = np.concatenate([v_cache, v], axis=2)
    if num_cond_latents:
        T, Hl, Wl = latent_shape
        q_pad = np.concatenate([np.zeros_like(k_cache), q], axis=2)
        f = B.rope_freqs_3d((T + num_cond_latents, Hl, Wl), D).astype(F32)
        cos, sin = np.cos(f), np.sin(f)
        q_pad = B.round_to(q_pad * cos + B.rotate_half(q_pad) * sin, dtype)
        k_full = B.round_to(k_full * cos + B.rotate_half(k_full) * sin, dtype)
        q = q_pad[:, :, -N:]
    gq, gk = bsa.get("noise") or (None, None)
    o, idx = _branch(q, k_full, v_full, gq, gk, bsa["top_k"], (block_indices or {}).get("noise"))
    o = np.transpose(_r(o, dtype), (0, 2, 1, 3)).reshape(Bsz, N, C)
    return linear(o, p["attn.proj.weight"], p["attn.proj.bias"], dtype), {"noise": idx}


def cross_attention(x, y, p, num_heads: int, dtype: str, num_cond_latents: int = 0, latent_shape=None):
    """MultiHeadCrossAttention (attention.py:300-371) for one batch item (x
    [1, N, C], text y [1, L, C]): q / kv projections, q_norm / k_norm, dense
    attention, proj.  With conditioning latents only the noise tokens attend
    and the conditioning rows are zero."""
    if num_cond_latents:
        nc = x.shape[1] // latent_shape[0] * num_cond_latents
        out = cross_attention(x[:, nc:], y, p, num_heads, dtype)
        return np.concatenate([np.zeros((x.shape[0], nc, x.shape[2]), F32), out], axis=1)
    Bsz, N, C = x.shape
    H, D = num_heads, C // num_heads
    q = linear(x, p["cross_attn.q_linear.weight"], p["cross_attn.q_linear.bias"], dtype).reshape(Bsz, N, H, D)
    kv = linear(y, p["cross_attn.kv_linear.weight"], p["cross_attn.kv_linear.bias"], dtype)
    kv = kv.reshape(Bsz, -1, 2, H, D)
    k, v = kv[:, :, 0], kv[:, :, 1]
    q = B.rms_norm_fp32(q, p["cross_attn.q_norm.weight"], 1e-6, dtype)
    k = B.rms_norm_fp32(k, p["cross_attn.k_norm.weight"], 1e-6, dtype)
    q, k, v = (np.transpose(a, (0, 2, 1, 3)) for a in (q, k, v))
    o = _r(dense_attention(q, k, v, D ** -0.5), dtype)
    o = np.transpose(o, (0, 2, 1, 3)).reshape(Bsz, N, C)
    return linear(o, p["cross_attn.proj.weight"], p["cross_attn.proj.bias"], dtype)


def dit_block(x, y, t, p, latent_shape: Sequence[int], num_heads: int, dtype: str, bsa: dict,
              block_indices=None, num_cond_latents: int = 0):
    """LongCatSingleStreamBlock.__call__ (longcat_video_dit.py:80-138) without
    a KV cache, cross-attention on.  x [B, N, C] (model dtype), y [1, L, C]
    text, t [B, T, Ct] fp32 timestep embedding; ``bsa`` / ``block_indices``
    as in ``self_attention``.  Returns (x_out, routing per branch)."""
    x = np.asarray(x, F32)
    Bsz, N, C = x.shape
    T = latent_shape[0]
    ada = silu(t) @ np.asarray(p["adaLN_modulation.1.weight"], np.float64).T + np.asarray(
        p["adaLN_modulation.1.bias"], np.float64)
    ada = ada.astype(F32)[:, :, None, :]
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = np.split(ada, 6, axis=-1)

    x_m = modulate_fp32(x.reshape(Bsz, T, -1, C), shift_msa, scale_msa, dtype).reshape(Bsz, N, C)
    x_s, idx = self_attention(x_m, p, latent_shape, num_heads, dtype, bsa, block_indices, num_cond_latents)
    x = _r(x.astype(np.float64) + (gate_msa.astype(np.float64) * x_s.reshape(Bsz, T, -1, C)).reshape(Bsz, N, C),
           dtype)

    xn = _r(layer_norm_fp32(x, p["pre_crs_attn_norm.weight"], p["pre_crs_attn_norm.bias"]), dtype)
    x = _r(x.astype(np.float64) + cross_attention(xn, y, p, num_heads, dtype, num_cond_latents, latent_shape),
           dtype)

    x_m = modulate_fp32(x.reshape(Bsz, T, -1, C), shift_mlp, scale_mlp, dtype).reshape(Bsz, N, C)
    x_s = feed_forward_swiglu(x_m, p["ffn.w1.weight"], p["ffn.w2.weight"], p["ffn.w3.weight"], dtype)
    x = _r(x.astype(np.float64) + (gate_mlp.astype(np.float64) * x_s.reshape(Bsz, T, -1, C)).reshape(Bsz, N, C),
           dtype)
    return x, idx


def block_param_shapes(hidden: int, num_heads: int, mlp_ratio: int = 4, t_dim: int = 512) -> dict:
    """Parameter names and shapes of one block (the PyTorch checkpoint keys)."""
    C, D, Hf = hidden, hidden // num_heads, swiglu_hidden_dim(hidden * mlp_ratio)
    return {
        "adaLN_modulation.1.weight": (6 * C, t_dim), "adaLN_modulation.1.bias": (6 * C,),
        "pre_crs_attn_norm.weight": (C,), "pre_crs_attn_norm.bias": (C,),
        "attn.qkv.weight": (3 * C, C), "attn.qkv.bias": (3 * C,),
        "attn.q_norm.weight": (D,), "attn.k_norm.weight": (D,),
        "attn.proj.weight": (C, C), "attn.proj.bias": (C,),
        "cross_attn.q_linear.weight": (C, C), "cross_attn.q_linear.bias": (C,),
        "cross_attn.kv_linear.weight": (2 * C, C), "cross_attn.kv_linear.bias": (2 * C,),
        "cross_attn.proj.weight": (C, C), "cross_attn.proj.bias": (C,),
        "cross_attn.q_norm.weight": (D,), "cross_attn.k_norm.weight": (D,),
        "ffn.w1.weight": (Hf, C), "ffn.w2.weight": (C, Hf), "ffn.w3.weight": (Hf, C),
    }
