"""3D rotary position embedding on torch tensors.

Restates ``RotaryPositionalEmbedding`` (longcat_video/models/rope_3d.py:37-128):
the head dim splits into t / h / w parts of ``D - 4*(D//6)``, ``2*(D//6)``,
``2*(D//6)`` dims (44 / 42 / 42 at D=128, rope_3d.py:60-62); each part uses
inverse frequencies ``1 / 10000^(2i/dim)`` (:65-70) at integer grid
positions (:80-82), every frequency repeated for an adjacent pair (:91-93),
and ``x*cos + rotate_half(x)*sin`` is applied in fp32 (:120-128) with
``rotate_half`` mapping each pair (a, b) to (-b, a) (:23-34).

RoPE is applied to q and k before BSA in the DiT (attention.py:201); here it
builds the benchmark inputs of the refinement shapes.
"""

from __future__ import annotations

import torch

__all__ = ["rope_dims", "rope_freqs_3d", "rotate_half", "apply_rope", "rope_3d"]

BASE = 10000.0


def rope_dims(head_dim: int) -> tuple[int, int, int]:
    """(dim_t, dim_h, dim_w), rope_3d.py:60-62."""
    assert head_dim % 8 == 0, "head_dim must be a multiple of 8 for 3D RoPE"
    return head_dim - 4 * (head_dim // 6), 2 * (head_dim // 6), 2 * (head_dim // 6)


def _axis_freqs(dim: int, n: int, device) -> torch.Tensor:
    idx = torch.arange(0, dim, 2, dtype=torch.float32, device=device)[: dim // 2]
    inv = 1.0 / (BASE ** (idx / dim))
    pos = torch.arange(0, n, dtype=torch.float32, device=device)
    return torch.repeat_interleave(pos[:, None] * inv[None, :], 2, dim=-1)  # (n, dim)


def rope_freqs_3d(grid: tuple[int, int, int], head_dim: int, device=None) -> torch.Tensor:
    """Per-token angles ``[T*H*W, head_dim]`` (fp32), t-major token order."""
    T, H, W = grid
    dt, dh, dw = rope_dims(head_dim)
    ft = _axis_freqs(dt, T, device)[:, None, None, :].expand(T, H, W, dt)
    fh = _axis_freqs(dh, H, device)[None, :, None, :].expand(T, H, W, dh)
    fw = _axis_freqs(dw, W, device)[None, None, :, :].expand(T, H, W, dw)
    return torch.cat([ft, fh, fw], dim=-1).reshape(T * H * W, head_dim)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """Pairs (a, b) -> (-b, a) along the last axis (rope_3d.py:23-34)."""
    x2 = x.reshape(*x.shape[:-1], x.shape[-1] // 2, 2)
    return torch.stack([-x2[..., 1], x2[..., 0]], dim=-1).reshape(x.shape)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """``x*cos + rotate_half(x)*sin`` in fp32; returns fp32."""
    xf = x.float()
    return xf * cos + rotate_half(xf) * sin


def rope_3d(q: torch.Tensor, k: torch.Tensor, grid: tuple[int, int, int]):
    """Rotate q, k ``[B, H, S, D]`` over ``grid``; returns them in their dtype."""
    f = rope_freqs_3d(grid, q.shape[-1], q.device)
    cos, sin = torch.cos(f), torch.sin(f)
    return apply_rope(q, cos, sin).to(q.dtype), apply_rope(k, cos, sin).to(k.dtype)
