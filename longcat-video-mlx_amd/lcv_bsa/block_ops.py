"""Fused row operations of the DiT block (HIP), with torch tensors.

``residual_norm`` covers the block's AdaLN modulation, gated residuals and
the cross-attention pre-norm (longcat_video_dit.py:107-136; blocks.py:
79-119), ``swiglu`` the SwiGLU gate (blocks.py:50-51) and ``head_rms_norm``
the cross-attention's per-head q / k norms (attention.py:325-326).  Each is
one pass over HBM through ``liblcv_bsa.so``; each rounds like the
reference's sequence of fp32 tensor operations followed by a cast.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib
from .block_sparse_attention import _dtype_code, _require_device, _stream, _strides

__all__ = ["residual_norm", "swiglu", "head_rms_norm"]


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _rows(t: torch.Tensor, name: str, shape) -> torch.Tensor:
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must be {tuple(shape)}, got {tuple(t.shape)}")
    return t.contiguous()


def residual_norm(
    x: torch.Tensor,
    a: Optional[torch.Tensor] = None,
    gate: Optional[torch.Tensor] = None,
    *,
    frames: int,
    shift: Optional[torch.Tensor] = None,
    scale: Optional[torch.Tensor] = None,
    weight: Optional[torch.Tensor] = None,
    bias: Optional[torch.Tensor] = None,
    eps: float = 1e-6,
    residual: bool = True,
    norm: bool = True,
):
    """``x``, ``a``: ``[B, N, C]`` fp16 / bf16.  Forms ``r = x``, ``x + a`` or
    ``x + gate * a`` (gate fp32 ``[B, frames, C]`` or ``[B, frames, 1, C]``),
    and ``LayerNorm(r)`` with the affine ``weight`` / ``bias`` or the AdaLN
    ``shift`` / ``scale`` (fp32, per frame).  Returns ``(r, n)`` (each None
    when not asked for; ``r`` is ``x`` itself when ``a`` is None)."""
    _require_device(x)
    B, N, C = x.shape
    x = x.contiguous()
    fshape = (B, frames, C)

    def per_frame(t, name):
        if t is None:
            return None
        t = t.reshape(t.shape[0], t.shape[1], -1) if t.dim() == 4 else t
        if t.dtype != torch.float32:
            raise ValueError(f"{name} must be fp32")
        return _rows(t, name, fshape)

    a = None if a is None else _rows(a, "a", x.shape)
    gate, shift, scale = per_frame(gate, "gate"), per_frame(shift, "shift"), per_frame(scale, "scale")
    if weight is not None:
        weight = _rows(weight.to(x.dtype), "weight", (C,))
        bias = _rows(bias.to(x.dtype), "bias", (C,))
    r = torch.empty_like(x) if (a is not None and residual) else None
    n = torch.empty_like(x) if norm else None
    st = _lib.load().lcv_bsa_block_rows(
        x.data_ptr(), _ptr(a), _dtype_code(x), B, N, C, int(frames), _ptr(gate), _ptr(shift), _ptr(scale),
        _ptr(weight), _ptr(bias), float(eps), _ptr(r), _ptr(n), _stream(x))
    _lib.check(st, "residual_norm")
    return (x if a is None else r), n


def swiglu(h13: torch.Tensor) -> torch.Tensor:
    """``h13``: ``[..., 2 * hidden]`` (w1 output then w3 output) ->
    ``silu(h1) * h3`` of shape ``[..., hidden]``."""
    _require_device(h13)
    h = h13.contiguous()
    hidden = h.shape[-1] // 2
    rows = h.numel() // h.shape[-1]
    out = torch.empty((*h.shape[:-1], hidden), dtype=h.dtype, device=h.device)
    st = _lib.load().lcv_bsa_block_swiglu(h.data_ptr(), _dtype_code(h), rows, hidden, out.data_ptr(), _stream(h))
    _lib.check(st, "swiglu")
    return out


def head_rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float = 1e-6,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """RMSNorm_FP32 over the last dim of a ``[B, H, S, D]`` view (any strides
    with dense D) into ``out`` (default: contiguous ``[B, H, S, D]``)."""
    _require_device(x)
    B, H, S, D = x.shape
    if out is None:
        out = torch.empty((B, H, S, D), dtype=x.dtype, device=x.device)
    if weight is not None:
        weight = _rows(weight.to(x.dtype), "weight", (D,))
    st = _lib.load().lcv_bsa_head_rms_norm(
        x.data_ptr(), _dtype_code(x), B, H, S, D, _strides(x), _ptr(weight), float(eps),
        out.data_ptr(), _strides(out), _stream(x))
    _lib.check(st, "head_rms_norm")
    return out
