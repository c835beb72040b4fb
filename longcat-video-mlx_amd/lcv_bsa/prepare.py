"""Pre-BSA preparation of q and k: RMSNorm + 3D RoPE + block means, in one pass.

In the DiT's attention layer the BSA inputs are produced by
(longcat_video/models/attention.py:191-201)::

    q, k, v = split(qkv(x))            # [B, H, N, D] views of the QKV output
    q = self.q_norm(q); k = self.k_norm(k)   # RMSNorm_FP32(head_dim, eps=1e-6)
    q, k = self.rope_3d(q, k, shape)

and BSA then pools q and k per block (block_sparse_attention.py:98-104).
``prepare_qk`` does all of it in one HIP pass over q and k
(``lcv_bsa_prepare_qk``), returning the prepared q, k and their fp32 block
means, which ``bsa_attention(..., block_means=(qbar, kbar))`` consumes
instead of pooling again.

RMSNorm_FP32 (longcat_video/models/blocks.py:55-72): ``x * rsqrt(mean(x^2) +
eps)`` in fp32, rounded to the input dtype, then multiplied by the weight in
that dtype.  rope_3d (rope_3d.py:107-128): widened to fp32,
``x*cos + rotate_half(x)*sin``, rounded back.  The cos / sin table is built
here with the reference's angle formula (rope_3d.py:65-93).
"""

from __future__ import annotations

from typing import Optional, Sequence

import torch

from . import _lib
from .block_sparse_attention import (
    _aligned_rows, _bhsd, _check_shape, _dtype_code, _geom, _require_device, _stream, _strides,
    num_blocks,
)
from .rope_3d import BASE, rope_dims

__all__ = ["rope_table", "prepare_qk", "RMS_EPS"]

RMS_EPS = 1e-6  # q_norm / k_norm, attention.py:53-54


def _axis_table(dim: int, n: int, device) -> tuple[torch.Tensor, torch.Tensor]:
    idx = torch.arange(0, dim, 2, dtype=torch.float32, device=device)[: dim // 2]
    inv = 1.0 / (BASE ** (idx / dim))
    ang = torch.arange(0, n, dtype=torch.float32, device=device)[:, None] * inv[None, :]
    return torch.cos(ang).reshape(-1), torch.sin(ang).reshape(-1)


_TABLES: dict = {}


def rope_table(head_dim: int, grid: Sequence[int], device=None) -> torch.Tensor:
    """The per-axis cos / sin table of ``lcv_bsa_prepare_qk`` (fp32, flat):
    cos_t, sin_t [T, dt/2], cos_h, sin_h [Hl, dh/2], cos_w, sin_w [Wl, dw/2].

    Built once per (head_dim, grid, device) and kept: the kernel only reads
    it, and building it takes about thirty small launches (~0.15 ms at
    720p), which would otherwise recur in every attention layer."""
    dev = torch.device(device) if device is not None else torch.device("cpu")
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    key = (int(head_dim), tuple(int(x) for x in grid), dev)
    table = _TABLES.get(key)
    if table is None:
        table = _TABLES[key] = _build_table(head_dim, grid, dev)
    return table


def _build_table(head_dim: int, grid: Sequence[int], device) -> torch.Tensor:
    T, Hl, Wl = (int(x) for x in grid)
    dt, dh, dw = rope_dims(head_dim)
    parts = []
    for dim, n in ((dt, T), (dh, Hl), (dw, Wl)):
        parts.extend(_axis_table(dim, n, device))
    return torch.cat(parts).contiguous()


def prepare_qk(
    q: torch.Tensor,
    k: torch.Tensor,
    grid: Sequence[int],
    *,
    q_weight: Optional[torch.Tensor] = None,
    k_weight: Optional[torch.Tensor] = None,
    eps: float = RMS_EPS,
    shape: Optional[Sequence[int]] = None,
    chunk_thw: Sequence[int] = (4, 4, 4),
):
    """RMSNorm + 3D RoPE of q and k (``[B, H, S, D]``, fp16 / bf16, any row
    strides) over the latent ``grid`` (T, H, W), plus their block means for
    the BSA geometry ``shape`` / ``chunk_thw`` (``shape`` defaults to
    ``grid``; blocks must hold 64 tokens).

    Returns ``(q_out, k_out, q_blocks, k_blocks)``: contiguous q, k in the
    input dtype and fp32 ``[B, H, nb, D]`` means.
    """
    _require_device(q, k)
    q, k = _bhsd(q, "q"), _bhsd(k, "k")
    if q.shape != k.shape or q.dtype != k.dtype:
        raise ValueError("q and k must share shape and dtype")
    B, H, S, D = q.shape
    shape = tuple(grid) if shape is None else tuple(shape)
    _check_shape(S, shape, chunk_thw)
    code = _dtype_code(q)
    q, k = _aligned_rows(q), _aligned_rows(k)
    weights = []
    for w in (q_weight, k_weight):
        if w is None:
            weights.append(None)
            continue
        if w.shape != (D,):
            raise ValueError(f"norm weight must be [{D}], got {tuple(w.shape)}")
        weights.append(w.to(device=q.device, dtype=q.dtype).contiguous())
    lib = _lib.load()
    g = _lib.Grid(*(int(x) for x in grid))
    n_tab = lib.lcv_bsa_rope_table_len(D, g)
    if n_tab == 0:
        raise ValueError(f"prepare_qk supports D in {{64, 128}} and RoPE grids up to the table limit "
                         f"(D={D}, grid={tuple(grid)})")
    table = rope_table(D, grid, q.device)
    assert table.numel() == n_tab
    nb = num_blocks(shape, chunk_thw)
    q_out = torch.empty((B, H, S, D), dtype=q.dtype, device=q.device)
    k_out = torch.empty_like(q_out)
    q_blocks = torch.empty((B, H, nb, D), dtype=torch.float32, device=q.device)
    k_blocks = torch.empty_like(q_blocks)
    st = lib.lcv_bsa_prepare_qk(
        q.data_ptr(), k.data_ptr(), code, B, H, S, D, _strides(q), _strides(k),
        weights[0].data_ptr() if weights[0] is not None else None,
        weights[1].data_ptr() if weights[1] is not None else None,
        float(eps), g, table.data_ptr(), n_tab, _geom(shape, chunk_thw),
        q_out.data_ptr(), k_out.data_ptr(), _strides(q_out), _strides(k_out),
        q_blocks.data_ptr(), k_blocks.data_ptr(), _stream(q),
    )
    _lib.check(st, "prepare_qk")
    return q_out, k_out, q_blocks, k_blocks
