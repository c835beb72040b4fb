"""One LongCat-Video DiT block on PyTorch-ROCm with the HIP attention path.

Mirrors ``LongCatSingleStreamBlock`` (longcat_video/models/
longcat_video_dit.py:36-138) and its parts (blocks.py:23-119,
attention.py:40-371) with the reference's module and parameter names, so a
PyTorch checkpoint's block keys load unchanged.  The linear layers are
torch GEMMs (hipBLASLt); the self-attention runs the library's fused pre-BSA
pass (RMSNorm + 3D RoPE + block means, ``prepare_qk``) and BSA routed from
those means, writing straight into the ``[B, N, H, D]`` layout the output
projection reads.  AdaLN modulation and the gated residuals stay in fp32 as
in the reference.

The block covers the reference's paths: text-to-video, conditioning latents
(image-to-video / continuation), returning the KV cache and continuing from
it; the cross-attention handles any batch with per-item text lengths.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import BSAAttention, dense_attention, validate_backend
from .block_ops import head_rms_norm, residual_norm, swiglu
from .block_sparse_attention import bsa_attention
from .block_sparse_attention_hip import bsa_attention_hip
from .prepare import prepare_qk
from .rope_3d import rope_3d
from .shape_policy import bsa_geometry

__all__ = [
    "RMSNorm_FP32", "LayerNorm_FP32", "modulate_fp32", "FeedForwardSwiGLU", "Attention",
    "MultiHeadCrossAttention", "LongCatSingleStreamBlock",
]


class RMSNorm_FP32(nn.Module):
    """``(x_f32 * rsqrt(mean(x_f32^2) + eps)).to(x.dtype) * weight`` (blocks.py:55-72)."""

    def __init__(self, dim: int, eps: float, **kw):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, **kw))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)).to(x.dtype) * self.weight


class LayerNorm_FP32(nn.Module):
    """LayerNorm computed in fp32, cast back to the input dtype (blocks.py:79-103)."""

    def __init__(self, dim: int, eps: float, elementwise_affine: bool, **kw):
        super().__init__()
        self.dim, self.eps = dim, eps
        self.elementwise_affine = elementwise_affine
        if elementwise_affine:
            self.weight = nn.Parameter(torch.ones(dim, **kw))
            self.bias = nn.Parameter(torch.zeros(dim, **kw))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        w = self.weight.float() if self.elementwise_affine else None
        b = self.bias.float() if self.elementwise_affine else None
        return F.layer_norm(x.float(), (self.dim,), w, b, self.eps).to(x.dtype)


def modulate_fp32(norm: LayerNorm_FP32, x: torch.Tensor, shift: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """``norm(x.float()) * (scale + 1) + shift`` in fp32, cast to x's dtype
    (blocks.py:106-119); shift / scale must be fp32."""
    assert shift.dtype == torch.float32 and scale.dtype == torch.float32, (
        f"modulate_fp32 takes fp32 shift and scale (got {shift.dtype} and {scale.dtype}): "
        "the AdaLN modulation is computed in fp32")
    return (norm(x.float()) * (scale + 1) + shift).to(x.dtype)


class FeedForwardSwiGLU(nn.Module):
    """``w2(silu(w1 x) * w3 x)``; inner width by the 2/3 rule rounded up to
    ``multiple_of`` (blocks.py:23-51): 11008 for dim 4096."""

    def __init__(self, dim: int, hidden_dim: int, multiple_of: int = 256,
                 ffn_dim_multiplier: Optional[float] = None, **kw):
        super().__init__()
        hidden_dim = int(2 * hidden_dim / 3)
        if ffn_dim_multiplier is not None:
            hidden_dim = int(ffn_dim_multiplier * hidden_dim)
        hidden_dim = multiple_of * ((hidden_dim + multiple_of - 1) // multiple_of)
        self.dim, self.hidden_dim = dim, hidden_dim
        self.w1 = nn.Linear(dim, hidden_dim, bias=False, **kw)
        self.w2 = nn.Linear(hidden_dim, dim, bias=False, **kw)
        self.w3 = nn.Linear(dim, hidden_dim, bias=False, **kw)

        self.fused = True            # on the GPU: one w1|w3 GEMM + the HIP gate kernel
        self._w13 = None
        self._w13_key = None

    def _w13_weight(self) -> torch.Tensor:
        key = (self.w1.weight.data_ptr(), self.w1.weight._version, self.w3.weight.data_ptr(),
               self.w3.weight._version)
        if self._w13_key != key:
            self._w13 = torch.cat([self.w1.weight, self.w3.weight], 0).detach()
            self._w13_key = key
        return self._w13

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.fused and x.is_cuda and self.hidden_dim % 8 == 0:
            return self.w2(swiglu(F.linear(x, self._w13_weight())))
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class Attention(nn.Module, BSAAttention):
    """Self-attention with 3D RoPE and the BSA dispatch (attention.py:40-276):
    the plain path, the conditioning split (``num_cond_latents``) and the
    KV-cache continuation.

    BSA geometry comes from ``bsa_shape_policy`` (``"reference"`` keeps the
    reference's dense fallback when the voxel does not tile the grid;
    ``"auto"`` / ``"contiguous"`` use 64-token runs instead).  Where queries
    and keys differ in length -- the noise queries over conditioning + noise
    keys (attention.py:218-221) and the KV-cache continuation (273) -- the
    reference always runs dense attention; ``bsa_cond_noise = True`` runs BSA
    there too (k-blocks over the longer key grid).

    With BSA on and no KV cache to return, q and k go through one
    ``prepare_qk`` over the strided views of the QKV output (RMSNorm + RoPE +
    block means), and the attention writes straight into the ``[B, N, H, D]``
    layout of the output projection.  A ``ValueError`` anywhere on that path
    falls back to the reference's unfused sequence."""

    def __init__(self, dim: int, num_heads: int, **kw):
        nn.Module.__init__(self)
        BSAAttention.__init__(self, dim, num_heads)
        self.qkv = nn.Linear(dim, dim * 3, bias=True, **kw)
        self.q_norm = RMSNorm_FP32(self.head_dim, eps=1e-6, **kw)
        self.k_norm = RMSNorm_FP32(self.head_dim, eps=1e-6, **kw)
        self.proj = nn.Linear(dim, dim, **kw)
        self.bsa_shape_policy: str = "reference"
        self.bsa_cond_noise: bool = False
        self.keep_indices: bool = False          # store the last routing per branch (tests)
        self.last_indices: dict = {}
        self.last_paths: dict = {}

    def _attend(self, name, q, k, v, q_shape, kv_shape=None, means=None, out=None):
        """BSA over the policy's geometry for ``q_shape`` (and ``kv_shape``
        when k / v are longer), else dense; writes into ``out`` if given."""
        path = "dense"
        if self.enable_bsa and q_shape is not None and (kv_shape is None or self.bsa_cond_noise):
            validate_backend(self.bsa_backend)
            gq = bsa_geometry(q_shape, self.bsa_chunk_thw, self.bsa_shape_policy)
            gk = gq if kv_shape is None else bsa_geometry(kv_shape, self.bsa_chunk_thw, self.bsa_shape_policy)
            if gq is not None and gk is not None and gq[1] == gk[1]:
                try:
                    o, idx = bsa_attention(q, k, v, gq[0], sparsity=self.bsa_sparsity, chunk_thw=gq[1],
                                           sm_scale=self.scale, top_k=self.bsa_top_k, return_indices=True,
                                           block_means=means, out=out,
                                           kv_shape=None if kv_shape is None else gk[0])
                    if self.keep_indices:
                        self.last_indices[name] = idx
                    path = "bsa"
                except ValueError:
                    pass
        if path == "dense":
            o = dense_attention(q, k, v, self.scale)
            if out is not None:
                out.copy_(o)
                o = out
        self.last_paths[name] = path
        self.last_path = path
        return o

    def _split(self, q, k, v, shape, ncl, o):
        """The conditioning split (attention.py:202-221) into ``o`` [B, N, H, D]."""
        T, Hl, Wl = (int(s) for s in shape)
        nc = q.shape[2] // T * ncl
        self._attend("cond", q[:, :, :nc], k[:, :, :nc], v[:, :, :nc], (ncl, Hl, Wl),
                     out=o[:, :nc].transpose(1, 2))
        self._attend("noise", q[:, :, nc:], k, v, (T - ncl, Hl, Wl), kv_shape=(T, Hl, Wl),
                     out=o[:, nc:].transpose(1, 2))

    def forward(self, x: torch.Tensor, shape: Sequence[int], num_cond_latents: Optional[int] = None,
                return_kv: bool = False):
        B, N, C = x.shape
        H, D = self.num_heads, self.head_dim
        ncl = int(num_cond_latents or 0)
        self.last_indices, self.last_paths = {}, {}
        qkv = self.qkv(x).view(B, N, 3, H, D)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        o = torch.empty((B, N, H, D), dtype=x.dtype, device=x.device)
        if self.enable_bsa and shape is not None and not return_kv:
            validate_backend(self.bsa_backend)
            geom = bsa_geometry(shape, self.bsa_chunk_thw, self.bsa_shape_policy)
            if geom is not None:
                try:
                    qp, kp, qb, kb = prepare_qk(q, k, shape, q_weight=self.q_norm.weight,
                                                k_weight=self.k_norm.weight, eps=self.q_norm.eps,
                                                shape=geom[0], chunk_thw=geom[1])
                    if ncl > 0:
                        self._split(qp, kp, v, shape, ncl, o)
                    else:
                        self._attend("all", qp, kp, v, shape, means=(qb, kb), out=o.transpose(1, 2))
                    return self.proj(o.view(B, N, C))
                except ValueError:
                    self.last_indices, self.last_paths = {}, {}
        # The reference's sequence: norms, (cache,) RoPE, then BSA-or-dense.
        q, k = self.q_norm(q), self.k_norm(k)
        cache = (k, v)
        q, k = rope_3d(q, k, tuple(shape))
        if ncl > 0:
            self._split(q, k, v, shape, ncl, o)
        else:
            self._attend("all", q, k, v, shape, out=o.transpose(1, 2))
        out = self.proj(o.view(B, N, C))
        return (out, cache) if return_kv else out

    def forward_with_kv_cache(self, x: torch.Tensor, shape: Sequence[int], num_cond_latents: Optional[int],
                              kv_cache: tuple) -> torch.Tensor:
        """Chunked continuation (attention.py:235-275): fresh k / v appended to
        the cached (normed, un-rotated) ones; with conditioning latents RoPE
        runs over the extended grid (q zero-padded to align positions); the
        noise queries then attend to all keys."""
        B, N, C = x.shape
        H, D = self.num_heads, self.head_dim
        qkv = self.qkv(x).view(B, N, 3, H, D)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        q, k = self.q_norm(q), self.k_norm(k)
        T, Hl, Wl = (int(s) for s in shape)
        k_cache, v_cache = kv_cache
        if k_cache.shape[0] == 1 and B > 1:
            k_cache = k_cache.expand(B, *k_cache.shape[1:])
            v_cache = v_cache.expand(B, *v_cache.shape[1:])
        k_full = torch.cat([k_cache, k], dim=2)
        v_full = torch.cat([v_cache, v], dim=2)
        ncl = int(num_cond_latents or 0)
        if ncl > 0:
            q_pad = torch.cat([torch.zeros_like(k_cache), q], dim=2)
            q_pad, k_full = rope_3d(q_pad, k_full, (T + ncl, Hl, Wl))
            q = q_pad[:, :, -N:]
        self.last_indices, self.last_paths = {}, {}
        Tk = k_full.shape[2] // (Hl * Wl)
        o = torch.empty((B, N, H, D), dtype=x.dtype, device=x.device)
        kv_shape = (Tk, Hl, Wl) if Tk * Hl * Wl == k_full.shape[2] else None
        if kv_shape is None:
            o.transpose(1, 2).copy_(dense_attention(q, k_full, v_full, self.scale))
            self.last_path = self.last_paths["noise"] = "dense"
        else:
            self._attend("noise", q, k_full, v_full, (T, Hl, Wl), kv_shape=kv_shape, out=o.transpose(1, 2))
        return self.proj(o.view(B, N, C))


class MultiHeadCrossAttention(nn.Module):
    """Text cross-attention (attention.py:282-371).  Each batch item's visual
    queries attend to its own slice of the packed text, which is what the
    reference's block-diagonal mask expresses."""

    def __init__(self, dim: int, num_heads: int, **kw):
        super().__init__()
        assert dim % num_heads == 0, "dim must be divisible by num_heads"
        self.dim, self.num_heads = dim, num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.q_linear = nn.Linear(dim, dim, **kw)
        self.kv_linear = nn.Linear(dim, dim * 2, **kw)
        self.proj = nn.Linear(dim, dim, **kw)
        self.q_norm = RMSNorm_FP32(self.head_dim, eps=1e-6, **kw)
        self.k_norm = RMSNorm_FP32(self.head_dim, eps=1e-6, **kw)
        # On the GPU, with 64-aligned token and text lengths: fused norms and
        # the library's attention kernel (dense over the text blocks).
        self.fused = True

    def forward(self, x: torch.Tensor, cond: torch.Tensor, kv_seqlen: Sequence[int],
                num_cond_latents: Optional[int] = None, shape: Optional[Sequence[int]] = None) -> torch.Tensor:
        """With conditioning latents only the noise tokens attend to the text;
        the conditioning rows of the result are zero (attention.py:355-371)."""
        if num_cond_latents:
            assert shape is not None
            B, N, C = x.shape
            nc = N // int(shape[0]) * int(num_cond_latents)
            out_noise = self._cross(x[:, nc:], cond, kv_seqlen)
            return torch.cat([out_noise.new_zeros((B, nc, C)), out_noise], dim=1)
        return self._cross(x, cond, kv_seqlen)

    def _cross_fused(self, x, cond, kv_seqlen):
        """q / k norms in place on the projections' rows, then the library's
        attention kernel with every text block listed (dense over the text),
        written in the [B, N, H, D] layout the projection reads."""
        B, N, C = x.shape
        H, D = self.num_heads, self.head_dim
        q = self.q_linear(x).view(B, N, H, D).transpose(1, 2)      # [B, H, N, D] view
        head_rms_norm(q, self.q_norm.weight, self.q_norm.eps, out=q)
        kv = self.kv_linear(cond).view(1, -1, 2, H, D)
        k = kv[:, :, 0].transpose(1, 2)
        head_rms_norm(k, self.k_norm.weight, self.k_norm.eps, out=k)
        v = kv[:, :, 1].transpose(1, 2)
        o = torch.empty((B, N, H, D), dtype=x.dtype, device=x.device)
        off = 0
        for b in range(B):
            n = int(kv_seqlen[b])
            nk = n // 64
            idx = torch.arange(nk, dtype=torch.int32, device=x.device).expand(1, H, N // 64, nk).contiguous()
            bsa_attention_hip(q[b:b + 1], k[:, :, off:off + n], v[:, :, off:off + n], idx, (1, 1, 64),
                              (1, 1, N), self.scale, out=o[b:b + 1].transpose(1, 2), kv_shape=(1, 1, n))
            off += n
        return self.proj(o.view(B, N, C))

    def _cross(self, x: torch.Tensor, cond: torch.Tensor, kv_seqlen: Sequence[int]) -> torch.Tensor:
        B, N, C = x.shape
        H, D = self.num_heads, self.head_dim
        if (self.fused and x.is_cuda and N % 64 == 0 and all(int(n) % 64 == 0 for n in kv_seqlen)
                and D in (64, 128) and x.dtype in (torch.float16, torch.bfloat16)):
            return self._cross_fused(x, cond, kv_seqlen)
        q = self.q_norm(self.q_linear(x).view(B, N, H, D)).transpose(1, 2).contiguous()
        kv = self.kv_linear(cond).view(1, -1, 2, H, D)
        k = self.k_norm(kv[:, :, 0]).transpose(1, 2).contiguous()
        v = kv[:, :, 1].transpose(1, 2).contiguous()
        outs, off = [], 0
        for b in range(B):
            n = int(kv_seqlen[b])
            outs.append(dense_attention(q[b:b + 1], k[..., off:off + n, :], v[..., off:off + n, :], self.scale))
            off += n
        o = torch.cat(outs, 0) if B > 1 else outs[0]
        return self.proj(o.transpose(1, 2).reshape(B, N, C))


class LongCatSingleStreamBlock(nn.Module):
    """Self-attention + text cross-attention + SwiGLU FFN with AdaLN-zero
    modulation of the self-attention and FFN (longcat_video_dit.py:36-138)."""

    def __init__(self, hidden_size: int, num_heads: int, mlp_ratio: int, adaln_tembed_dim: int, **kw):
        super().__init__()
        self.hidden_size = hidden_size
        self.adaLN_modulation = nn.Sequential(nn.SiLU(), nn.Linear(adaln_tembed_dim, 6 * hidden_size, bias=True, **kw))
        self.mod_norm_attn = LayerNorm_FP32(hidden_size, eps=1e-6, elementwise_affine=False)
        self.mod_norm_ffn = LayerNorm_FP32(hidden_size, eps=1e-6, elementwise_affine=False)
        self.pre_crs_attn_norm = LayerNorm_FP32(hidden_size, eps=1e-6, elementwise_affine=True, **kw)
        self.attn = Attention(hidden_size, num_heads, **kw)
        self.cross_attn = MultiHeadCrossAttention(hidden_size, num_heads, **kw)
        self.ffn = FeedForwardSwiGLU(hidden_size, int(hidden_size * mlp_ratio), **kw)
        # On the GPU: modulation, gated residuals and the pre-norm as fused
        # HIP row passes (same fp32 arithmetic as the unfused path below).
        self.fused = True

    def _self_attn(self, x_m, latent_shape, num_cond_latents, return_kv, kv_cache):
        if kv_cache is not None:
            return self.attn.forward_with_kv_cache(x_m, latent_shape, num_cond_latents, kv_cache), kv_cache
        if return_kv:
            return self.attn(x_m, latent_shape, num_cond_latents, return_kv=True)
        return self.attn(x_m, latent_shape, num_cond_latents), None

    def _forward_fused(self, x, y, t, y_seqlen, latent_shape, num_cond_latents, return_kv, kv_cache,
                       skip_crs_attn, ada):
        T = int(latent_shape[0])
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = ada.chunk(6, dim=-1)
        _, x_m = residual_norm(x, frames=T, shift=shift_msa, scale=scale_msa, eps=self.mod_norm_attn.eps)
        x_s, new_kv = self._self_attn(x_m, latent_shape, num_cond_latents, return_kv, kv_cache)
        pre = self.pre_crs_attn_norm
        x, xn = residual_norm(x, x_s, gate_msa, frames=T, weight=pre.weight, bias=pre.bias, eps=pre.eps,
                              norm=not skip_crs_attn)
        if not skip_crs_attn:
            ncl_cross = None if kv_cache is not None else num_cond_latents
            c = self.cross_attn(xn, y, y_seqlen, ncl_cross, latent_shape)
            x, x_m = residual_norm(x, c, frames=T, shift=shift_mlp, scale=scale_mlp, eps=self.mod_norm_ffn.eps)
        else:
            _, x_m = residual_norm(x, frames=T, shift=shift_mlp, scale=scale_mlp, eps=self.mod_norm_ffn.eps)
        x, _ = residual_norm(x, self.ffn(x_m), gate_mlp, frames=T, norm=False)
        return (x, new_kv) if return_kv else x

    def forward(self, x: torch.Tensor, y: torch.Tensor, t: torch.Tensor, y_seqlen: Sequence[int],
                latent_shape: Sequence[int], num_cond_latents: Optional[int] = None, return_kv: bool = False,
                kv_cache: Optional[tuple] = None, skip_crs_attn: bool = False):
        """x [B, N, C] visual tokens, y [1, sum(y_seqlen), C] packed text,
        t [B, T, C_t] fp32 timestep embedding, latent_shape (T, H, W).
        Returns x, or (x, kv) with ``return_kv`` (longcat_video_dit.py:80-138)."""
        dtype = x.dtype
        B, N, C = x.shape
        T = int(latent_shape[0])
        lin = self.adaLN_modulation[1]
        ada = F.linear(F.silu(t.float()), lin.weight.float(), lin.bias.float())[:, :, None, :]
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = ada.chunk(6, dim=-1)

        if self.fused and x.is_cuda and x.dtype in (torch.float16, torch.bfloat16) and C % 8 == 0:
            return self._forward_fused(x, y, t, y_seqlen, latent_shape, num_cond_latents, return_kv, kv_cache,
                                       skip_crs_attn, ada)
        x_m = modulate_fp32(self.mod_norm_attn, x.view(B, T, -1, C), shift_msa, scale_msa).view(B, N, C)
        x_s, new_kv = self._self_attn(x_m, latent_shape, num_cond_latents, return_kv, kv_cache)
        x = (x.float() + (gate_msa * x_s.view(B, T, -1, C).float()).view(B, N, C)).to(dtype)

        if not skip_crs_attn:
            ncl_cross = None if kv_cache is not None else num_cond_latents
            x = x + self.cross_attn(self.pre_crs_attn_norm(x), y, y_seqlen, ncl_cross, latent_shape)

        x_m = modulate_fp32(self.mod_norm_ffn, x.view(B, T, -1, C), shift_mlp, scale_mlp).view(B, N, C)
        x_s = self.ffn(x_m)
        x = (x.float() + (gate_mlp * x_s.view(B, T, -1, C).float()).view(B, N, C)).to(dtype)
        return (x, new_kv) if return_kv else x
