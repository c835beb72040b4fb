"""The DiT block oracle restated in torch fp32, for the full 720p size on the GPU.

TEST INFRASTRUCTURE ONLY.  The NumPy block oracle (oracle/dit_block_oracle.py)
evaluates its matrix products in fp64 and is far too slow for one block at
720p (57,600 tokens, hidden 4096: ~27 TFLOP).  This module follows the oracle
step for step -- the same rounding to the model dtype after every op that
produces a model-dtype tensor, fp32 AdaLN / modulation / gated residuals,
fp32 RoPE, BSA over given routing lists -- with fp32 torch matmuls, so it
runs on the GPU in seconds.  It shares no code with the product package;
test_oracle_dit_block.py::test_torch_block_reference_matches_oracle pins it
against the NumPy oracle on a small block.

Reference: LongCatSingleStreamBlock.__call__ (longcat_video/models/
longcat_video_dit.py:80-138), blocks.py:23-119, attention.py:186-233, 282-371.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from conftest import gathered_attention_fp32
from oracle import bsa_oracle as BO

__all__ = ["dit_block_torch"]


def _r(x: torch.Tensor, dt: torch.dtype) -> torch.Tensor:
    """Round fp32 values to the model dtype (nearest even) and widen back."""
    return x.to(dt).float()


def _linear(x, w, b, dt):
    y = torch.matmul(x, w.float().t().contiguous())
    if b is not None:
        y = y + b.float()
    return _r(y, dt)


def _rms(x, w, dt, eps=1e-6):
    y = _r(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps), dt)
    return _r(y * _r(w.float(), dt), dt)


def _layer_norm(x, w=None, b=None, eps=1e-6):
    return F.layer_norm(x, (x.shape[-1],), None if w is None else w.float(),
                        None if b is None else b.float(), eps)


def _rotate_half(x):
    x2 = x.reshape(*x.shape[:-1], -1, 2)
    return torch.stack((-x2[..., 1], x2[..., 0]), dim=-1).reshape(x.shape)


def _dense(q, k, v, scale, step=8192):
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    kt = k.transpose(-1, -2).contiguous()
    for s0 in range(0, q.shape[-2], step):
        p = torch.softmax(torch.matmul(q[..., s0:s0 + step, :].contiguous(), kt) * scale, dim=-1)
        out[..., s0:s0 + step, :] = torch.matmul(p, v.contiguous())
    return out


def dit_block_torch(x, y, t, p: dict, latent_shape, num_heads: int, dt: torch.dtype, idx: torch.Tensor,
                    envelope: bool = False):
    """One block (text-to-video, no KV cache, cross-attention on) with BSA
    over contiguous 64-token blocks routed by ``idx`` [B, H, N/64, top_k].
    ``x`` [B, N, C] and ``y`` [1, L, C] in the model dtype, ``t`` [B, T, Ct]
    fp32, ``p`` the block's state dict.  Returns fp32 values of the model
    dtype; with ``envelope`` also the elementwise sum of the magnitudes of
    the four terms added into the residual stream (input, gated attention,
    cross-attention, gated FFN), the scale of the rounding error an
    implementation that rounds at the same points may carry."""
    x = x.float()
    Bsz, N, C = x.shape
    T = int(latent_shape[0])
    H, D = num_heads, C // num_heads
    ada = torch.matmul(F.silu(t.float()), p["adaLN_modulation.1.weight"].float().t()) + p["adaLN_modulation.1.bias"].float()
    shift_msa, scale_msa, gate_msa, shift_mlp, scale_mlp, gate_mlp = ada[:, :, None, :].chunk(6, dim=-1)

    def modulate(z, shift, scale):
        zz = z.view(Bsz, T, -1, C)
        return _r(_layer_norm(zz) * (scale + 1.0) + shift, dt).view(Bsz, N, C)

    def gated(res, branch, gate):
        return _r((res.view(Bsz, T, -1, C) + gate * branch.view(Bsz, T, -1, C)).view(Bsz, N, C), dt)

    # self-attention (attention.py:186-233)
    x_m = modulate(x, shift_msa, scale_msa)
    qkv = _linear(x_m, p["attn.qkv.weight"], p["attn.qkv.bias"], dt).view(Bsz, N, 3, H, D)
    q, k, v = (qkv[:, :, i].transpose(1, 2) for i in range(3))
    q = _rms(q, p["attn.q_norm.weight"], dt)
    k = _rms(k, p["attn.k_norm.weight"], dt)
    f = torch.from_numpy(BO.rope_freqs_3d(tuple(int(s) for s in latent_shape), D).astype(np.float32)).to(x.device)
    cos, sin = torch.cos(f), torch.sin(f)
    q = _r(q * cos + _rotate_half(q) * sin, dt)
    k = _r(k * cos + _rotate_half(k) * sin, dt)
    o = _r(gathered_attention_fp32(q, k, v, idx, D ** -0.5), dt)
    x_s = _linear(o.transpose(1, 2).reshape(Bsz, N, C), p["attn.proj.weight"], p["attn.proj.bias"], dt)
    env = x.abs() + (gate_msa * x_s.view(Bsz, T, -1, C)).abs().view(Bsz, N, C)
    x = gated(x, x_s, gate_msa)

    # cross-attention (attention.py:282-371), one batch item, all text tokens
    xn = _r(_layer_norm(x, p["pre_crs_attn_norm.weight"], p["pre_crs_attn_norm.bias"]), dt)
    cq = _linear(xn, p["cross_attn.q_linear.weight"], p["cross_attn.q_linear.bias"], dt).view(Bsz, N, H, D)
    kv = _linear(y.float(), p["cross_attn.kv_linear.weight"], p["cross_attn.kv_linear.bias"], dt)
    kv = kv.view(Bsz, -1, 2, H, D)
    ck, cv = kv[:, :, 0], kv[:, :, 1]
    cq = _rms(cq, p["cross_attn.q_norm.weight"], dt).transpose(1, 2)
    ck = _rms(ck, p["cross_attn.k_norm.weight"], dt).transpose(1, 2)
    co = _r(_dense(cq, ck, cv.transpose(1, 2), D ** -0.5), dt)
    c = _linear(co.transpose(1, 2).reshape(Bsz, N, C), p["cross_attn.proj.weight"], p["cross_attn.proj.bias"], dt)
    env = env + c.abs()
    x = _r(x + c, dt)

    # SwiGLU FFN (blocks.py:23-51)
    x_m = modulate(x, shift_mlp, scale_mlp)
    a = _r(F.silu(_linear(x_m, p["ffn.w1.weight"], None, dt)), dt)
    g = _r(a * _linear(x_m, p["ffn.w3.weight"], None, dt), dt)
    x_s = _linear(g, p["ffn.w2.weight"], None, dt)
    out = gated(x, x_s, gate_mlp)
    if envelope:
        return out, env + (gate_mlp * x_s.view(Bsz, T, -1, C)).abs().view(Bsz, N, C)
    return out
