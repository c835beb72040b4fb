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

Scope: the text-to-video block (no KV cache, no conditioning latents); the
cross-attention handles any batch with per-item text lengths.
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import BSAAttention, dense_attention, validate_backend
from .block_sparse_attention import bsa_attention
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
        "Modulation params must be fp32; AdaLN math diverges in bf16.")
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

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class Attention(nn.Module, BSAAttention):
    """Self-attention with 3D RoPE and the BSA dispatch (attention.py:40-233,
    text-to-video path).

    With BSA on, the geometry comes from ``bsa_shape_policy`` (``"reference"``
    keeps the reference's dense fallback when the voxel does not tile the
    grid; ``"auto"`` / ``"contiguous"`` use 64-token runs instead).  The BSA
    path is one ``prepare_qk`` over the strided q / k views of the QKV output
    plus ``bsa_attention`` from the fused block means; a ``ValueError`` from
    it falls back to the unfused layer and dense attention, as the reference
    does."""

    def __init__(self, dim: int, num_heads: int, **kw):
        nn.Module.__init__(self)
        BSAAttention.__init__(self, dim, num_heads)
        self.qkv = nn.Linear(dim, dim * 3, bias=True, **kw)
        self.q_norm = RMSNorm_FP32(self.head_dim, eps=1e-6, **kw)
        self.k_norm = RMSNorm_FP32(self.head_dim, eps=1e-6, **kw)
        self.proj = nn.Linear(dim, dim, **kw)
        self.bsa_shape_policy: str = "reference"
        self.keep_indices: bool = False          # store the last routing (tests)
        self.last_indices: Optional[torch.Tensor] = None

    def _bsa(self, q, k, v, shape, geom):
        bshape, bchunk = geom
        B, H, N, D = q.shape
        qp, kp, qb, kb = prepare_qk(q, k, shape, q_weight=self.q_norm.weight, k_weight=self.k_norm.weight,
                                    eps=self.q_norm.eps, shape=bshape, chunk_thw=bchunk)
        o = torch.empty((B, N, H, D), dtype=q.dtype, device=q.device)
        _, idx = bsa_attention(qp, kp, v, bshape, sparsity=self.bsa_sparsity, chunk_thw=bchunk,
                               sm_scale=self.scale, top_k=self.bsa_top_k, return_indices=True,
                               block_means=(qb, kb), out=o.transpose(1, 2))
        self.last_indices = idx if self.keep_indices else None
        return o

    def forward(self, x: torch.Tensor, shape: Sequence[int]) -> torch.Tensor:
        B, N, C = x.shape
        qkv = self.qkv(x).view(B, N, 3, self.num_heads, self.head_dim)
        q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
        if self.enable_bsa and shape is not None:
            validate_backend(self.bsa_backend)
            geom = bsa_geometry(shape, self.bsa_chunk_thw, self.bsa_shape_policy)
            if geom is not None:
                try:
                    o = self._bsa(q, k, v, shape, geom)
                    self.last_path = "bsa"
                    return self.proj(o.view(B, N, C))
                except ValueError:
                    pass
        # The reference's sequence: norms, RoPE, then its BSA-or-dense dispatch.
        q, k = rope_3d(self.q_norm(q), self.k_norm(k), tuple(shape))
        o = self._process_attn(q, k, v, shape=shape)
        return self.proj(o.transpose(1, 2).reshape(B, N, C))


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

    def forward(self, x: torch.Tensor, cond: torch.Tensor, kv_seqlen: Sequence[int]) -> torch.Tensor:
        B, N, C = x.shape
        H, D = self.num_heads, self.head_dim
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

    def forward(self, x: torch.Tensor, y: torch.Tensor, t: torch.Tensor, y_seqlen: Sequence[int],
                latent_shape: Sequence[int]) -> torch.Tensor:
        """x [B, N, C] visual tokens, y [1, sum(y_seqlen), C] packed text,
        t [B, T, C_t] fp32 timestep embedding, latent_shape (T, H, W)."""
        dtype = x.dtype
        B, N, C = x.shape
        T = int(latent_shape[0])
        lin = self.adaLN_modulation[1]
        ada = F.linear(F.silu(t.float()), lin.weight.float(), lin.bias.float())[:, :, None, :]
        shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = ada.chunk(6, dim=-1)

        x_m = modulate_fp32(self.mod_norm_attn, x.view(B, T, -1, C), shift_msa, scale_msa).view(B, N, C)
        x_s = self.attn(x_m, latent_shape)
        x = (x.float() + (gate_msa * x_s.view(B, T, -1, C).float()).view(B, N, C)).to(dtype)

        x = x + self.cross_attn(self.pre_crs_attn_norm(x), y, y_seqlen)

        x_m = modulate_fp32(self.mod_norm_ffn, x.view(B, T, -1, C), shift_mlp, scale_mlp).view(B, N, C)
        x_s = self.ffn(x_m)
        return (x.float() + (gate_mlp * x_s.view(B, T, -1, C).float()).view(B, N, C)).to(dtype)
