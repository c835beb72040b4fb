"""Kernel-level BSA entry: sparse attention from precomputed block indices.

The HIP counterpart of the reference's Tier B wrappers
``bsa_attention_metal{,_v2,_v3,_v4}(q, k, v, block_indices, chunk_thw, shape)``
(longcat_video/models/block_sparse_attention_metal.py:224-295, 484-548,
729-810, 985-1046): same arguments, same ``ValueError`` contract, t-major
input and output.  The reference permutes q/k/v to block-major order and
back around its kernel (metal.py:185-221); the gfx950 kernel addresses voxel
rows directly, so no permutation pass runs.  The permutation itself is still
exposed (``reshape_to_block_major`` / ``reshape_from_block_major``).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _lib
from .block_sparse_attention import (
    _aligned_rows, _bhsd, _check_shape, _dtype_code, _geom, _require_device, _stream, _strides,
    num_blocks,
)

__all__ = [
    "bsa_attention_hip", "schedule_block_order", "reshape_to_block_major",
    "reshape_from_block_major",
]

MAX_SCHEDULED_BLOCKS = 4096


def schedule_block_order(block_indices: torch.Tensor, num_kv_blocks: Optional[int] = None) -> torch.Tensor:
    """Per-head launch order of the q-blocks (``[B, H, nq]`` int32 permutation).

    q-blocks are sorted by the first and middle entries of their routing
    lists, so that blocks whose ascending lists start together run together
    and re-use each other's K/V tiles from L2.  Any order gives the same
    attention output up to fp32 rounding (a q-block's launch slot sets where
    its walk over its list starts, which changes the summation order); for a
    given order the result is deterministic.  ``num_kv_blocks`` is the K/V
    block count the entries index (default: nq, the S_q == S_k case).
    nq <= 4096.
    """
    _require_device(block_indices)
    bi = block_indices.to(torch.int32).contiguous()
    B, H, nq, k = bi.shape
    nk = nq if num_kv_blocks is None else int(num_kv_blocks)
    order = torch.empty((B, H, nq), dtype=torch.int32, device=bi.device)
    st = _lib.load().lcv_bsa_schedule_kv(bi.data_ptr(), B, H, nq, nk, k, order.data_ptr(), _stream(bi))
    _lib.check(st, "schedule_block_order")
    return order


def bsa_attention_hip(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    block_indices: torch.Tensor,
    chunk_thw: tuple[int, int, int] = (4, 4, 4),
    shape: Optional[tuple[int, int, int]] = None,
    sm_scale: Optional[float] = None,
    *,
    out: Optional[torch.Tensor] = None,
    kv_shape: Optional[tuple[int, int, int]] = None,
) -> torch.Tensor:
    """Attend each q-block to the KV blocks listed in ``block_indices``.

    Args:
        q, k, v: ``[B, H, S, D]`` t-major (fp16 / bf16 / fp32).
        block_indices: ``[B, H, num_q_blocks, top_k]`` integer block ids
            (entries outside ``[0, num_blocks)`` are skipped).
        chunk_thw: voxel shape; its product must be 64.
        shape: ``(T, H, W)``; required, as in the reference.
        sm_scale: softmax scale, default ``1/sqrt(D)`` (the reference
            kernels hard-code that value, metal.py:114, 410, 636, 873).
        out: optional ``[B, H, S, D]`` destination in q's dtype with unit
            last stride and 16-byte aligned rows, e.g. the ``transpose(1, 2)``
            view of a ``[B, S, H, D]`` buffer, so the head merge after
            attention needs no copy.
        kv_shape: the latent grid of k / v when it differs from q's (k, v
            ``[B, H, S_k, D]``; ``block_indices`` then holds k/v block ids),
            e.g. noise queries over conditioning + noise keys.
    Returns: ``[B, H, S, D]`` in q's dtype (``out`` when given).
    """
    if shape is None:
        raise ValueError(
            "shape=(T_lat, H_lat, W_lat) is required for the HIP BSA kernel "
            "(it locates each block's voxel rows in the t-major sequence)"
        )
    _require_device(q, k, v, block_indices)
    q, k, v = _bhsd(q, "q"), _bhsd(k, "k"), _bhsd(v, "v")
    if kv_shape is None:
        if not (q.shape == k.shape == v.shape):
            raise ValueError("q, k, v must have the same shape")
    elif not (k.shape == v.shape and k.shape[:2] == q.shape[:2] and k.shape[3] == q.shape[3]):
        raise ValueError(f"k, v must be [B, H, S_k, D] matching q {tuple(q.shape)}: "
                         f"got {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    B, H, S, D = q.shape
    Sk = k.shape[2]
    kshape = tuple(shape) if kv_shape is None else tuple(kv_shape)
    BS = int(chunk_thw[0]) * int(chunk_thw[1]) * int(chunk_thw[2])
    if S % BS != 0:
        raise ValueError(f"S={S} must be a multiple of block_size={BS}.")
    if Sk % BS != 0:
        raise ValueError(f"S_k={Sk} must be a multiple of block_size={BS}.")
    if BS != 64:
        raise ValueError(f"the HIP BSA kernel requires block_size=64 (got {BS}).")
    _check_shape(S, shape, chunk_thw)
    _check_shape(Sk, kshape, chunk_thw)
    nb = num_blocks(shape, chunk_thw)
    bi = block_indices
    if bi.dim() != 4 or tuple(bi.shape[:3]) != (B, H, nb):
        raise ValueError(
            f"block_indices must be [B, H, num_q_blocks, top_k] = [{B}, {H}, {nb}, k], "
            f"got {tuple(bi.shape)}"
        )
    bi = bi.to(torch.int32).contiguous()
    top_k = bi.shape[3]
    if top_k < 1:
        raise ValueError("block_indices must list at least one block per q-block")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    code = _dtype_code(q)
    if code != _lib.F32:
        q, k, v = _aligned_rows(q), _aligned_rows(k), _aligned_rows(v)
    nk = num_blocks(kshape, chunk_thw)
    order = schedule_block_order(bi, nk) if nb <= MAX_SCHEDULED_BLOCKS else None
    out = _output(out, q)
    st = _lib.load().lcv_bsa_attn_fwd_kv(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), code, B, H, S, Sk, D,
        _strides(q), _strides(k), _strides(v), bi.data_ptr(),
        order.data_ptr() if order is not None else None, top_k, float(sm_scale),
        _geom(shape, chunk_thw), _geom(kshape, chunk_thw), out.data_ptr(), _strides(out), _stream(q),
    )
    _lib.check(st, "bsa_attention_hip")
    return out


def _output(out: Optional[torch.Tensor], q: torch.Tensor) -> torch.Tensor:
    """A fresh ``[B, H, S, D]`` output, or the caller's after checking it."""
    if out is None:
        return torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype or out.device != q.device:
        raise ValueError(f"out must be {tuple(q.shape)} {q.dtype} on {q.device}, got "
                         f"{tuple(out.shape)} {out.dtype} on {out.device}")
    if out.stride(-1) != 1:
        raise ValueError("out must have unit stride in its last dimension")
    return out


def _permute(x: torch.Tensor, shape, chunk_thw, inverse: int) -> torch.Tensor:
    _require_device(x)
    x = x.contiguous()
    B, H, S, D = x.shape
    _check_shape(S, shape, chunk_thw)
    out = torch.empty_like(x)
    st = _lib.load().lcv_bsa_permute_block_major(
        x.data_ptr(), _dtype_code(x), B, H, S, D, _geom(shape, chunk_thw), inverse,
        out.data_ptr(), _stream(x))
    _lib.check(st, "permute_block_major")
    return out


def reshape_to_block_major(x: torch.Tensor, shape, chunk_thw) -> torch.Tensor:
    """t-major ``[B,H,S,D]`` -> block-major (metal.py:185-205)."""
    return _permute(x, shape, chunk_thw, 0)


def reshape_from_block_major(x: torch.Tensor, shape, chunk_thw) -> torch.Tensor:
    """Inverse of :func:`reshape_to_block_major` (metal.py:208-221)."""
    return _permute(x, shape, chunk_thw, 1)
