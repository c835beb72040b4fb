"""Block Sparse Attention on MI355X: the reference's Tier A API, HIP backed.

Mirrors ``longcat_video/models/block_sparse_attention.py`` (function names,
argument meaning, ``ValueError`` contract) on PyTorch-ROCm tensors.  Every
function runs a gfx950 kernel from ``liblcv_bsa.so`` on the current torch
stream; inputs must live on a ROCm device and nothing here falls back to
another implementation.

Differences from the reference, all deliberate:

* pooled block means are fp32 whatever the input dtype (the reference keeps
  the input dtype, block_sparse_attention.py:104); routing scores are fp32;
* ``topk_block_indices`` returns each row's set in ascending block order
  (``mx.argpartition`` leaves the order unspecified, :133-134) and breaks
  exact score ties toward the lower block index;
* ``bsa_attention`` never materialises the ``[B, H, S, S]`` mask (:238-247):
  it attends only the routed blocks, which gives the same result because
  masked entries contribute exactly zero;
* ``top_k=`` overrides the reference's count rule
  ``max(1, int((1 - sparsity) * num_kv_blocks))`` (:127).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch

from . import _lib

__all__ = [
    "mean_pool_blocks_3d",
    "block_routing_scores",
    "topk_block_indices",
    "select_block_indices",
    "build_token_block_indices",
    "build_token_pair_mask",
    "bsa_attention",
    "num_selected_blocks",
    "num_blocks",
    "BSADeviceError",
]

_DTYPES = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16, torch.float32: _lib.F32}


# ---------------------------------------------------------------------------
# Argument plumbing
# ---------------------------------------------------------------------------

def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


class BSADeviceError(RuntimeError):
    """Tensors are not on (one) ROCm device.  Deliberately not a ValueError:
    the dispatcher's dense fallback must not hide it."""


def _require_device(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise BSADeviceError(
                "the HIP BSA backend needs tensors on a ROCm device "
                f"(got a tensor on {t.device})"
            )
    dev = ts[0].device
    for t in ts[1:]:
        if t.device != dev:
            raise BSADeviceError(f"tensors on different devices: {dev} and {t.device}")


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}; use float16, bfloat16 or float32") from None


def _bhsd(t: torch.Tensor, name: str) -> torch.Tensor:
    """A [B, H, S, D] view whose D axis is dense (copies only when it isn't)."""
    if t.dim() != 4:
        raise ValueError(f"{name} must be [B, H, S, D], got shape {tuple(t.shape)}")
    if t.stride(3) != 1 or any(s < 0 for s in t.stride()):
        t = t.contiguous()
    return t


def _aligned_rows(t: torch.Tensor) -> torch.Tensor:
    """Rows 16-byte aligned (what the MFMA kernel loads); copy otherwise."""
    vec = 16 // t.element_size()
    if t.data_ptr() % 16 or any(s % vec for s in t.stride()[:3]):
        t = t.contiguous()
        if t.data_ptr() % 16:
            t = t.clone()
    return t


def _strides(t: torch.Tensor) -> _lib.Strides:
    sb, sh, ss, _ = t.stride()
    return _lib.Strides(sb, sh, ss)


def _geom(shape: Sequence[int], chunk_thw: Sequence[int]) -> _lib.Geom:
    T, H_, W = (int(x) for x in shape)
    cT, cH, cW = (int(x) for x in chunk_thw)
    return _lib.Geom(T, H_, W, cT, cH, cW)


def _check_shape(S: int, shape: Sequence[int], chunk_thw: Sequence[int]) -> None:
    """The reference's shape contract (block_sparse_attention.py:84-96)."""
    T, H_, W = (int(x) for x in shape)
    cT, cH, cW = (int(x) for x in chunk_thw)
    if min(cT, cH, cW) <= 0 or min(T, H_, W) <= 0:
        raise ValueError(f"shape {tuple(shape)} and chunk_thw {tuple(chunk_thw)} must be positive")
    if T % cT or H_ % cH or W % cW:
        raise ValueError(
            f"Latent shape ({T}, {H_}, {W}) must be a multiple of "
            f"chunk_thw {tuple(chunk_thw)}; refinement padding should guarantee this."
        )
    if S != T * H_ * W:
        raise ValueError(f"S={S} doesn't match T*H*W={T * H_ * W} for shape {tuple(shape)}")


def num_blocks(shape: Sequence[int], chunk_thw: Sequence[int] = (4, 4, 4)) -> int:
    """Number of voxel blocks of a latent grid."""
    T, H_, W = shape
    cT, cH, cW = chunk_thw
    return (T // cT) * (H_ // cH) * (W // cW)


def num_selected_blocks(num_kv_blocks: int, sparsity: float) -> int:
    """The reference's count rule, block_sparse_attention.py:127 (floor)."""
    return max(1, int((1.0 - sparsity) * num_kv_blocks))


# ---------------------------------------------------------------------------
# Tier A API
# ---------------------------------------------------------------------------

def mean_pool_blocks_3d(
    x: torch.Tensor,
    shape: tuple[int, int, int],
    chunk_thw: tuple[int, int, int] = (4, 4, 4),
) -> torch.Tensor:
    """``[B, H, S, D]`` -> ``[B, H, num_blocks, D]`` fp32 block means.

    Same contract as block_sparse_attention.py:67-104 (blocks in
    ``(bt, bh, bw)`` order; ``ValueError`` on a non-multiple shape).
    """
    _require_device(x)
    x = _bhsd(x, "x")
    B, H, S, D = x.shape
    _check_shape(S, shape, chunk_thw)
    nb = num_blocks(shape, chunk_thw)
    out = torch.empty((B, H, nb, D), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    st = lib.lcv_bsa_pool(x.data_ptr(), _dtype_code(x), B, H, S, D, _strides(x),
                          _geom(shape, chunk_thw), out.data_ptr(), _stream(x))
    _lib.check(st, "mean_pool_blocks_3d")
    return out


def block_routing_scores(q_blocks: torch.Tensor, k_blocks: torch.Tensor) -> torch.Tensor:
    """``q_blocks @ k_blocks^T`` in fp32, unscaled (block_sparse_attention.py:107-112)."""
    _require_device(q_blocks, k_blocks)
    qb = q_blocks.float().contiguous()
    kb = k_blocks.float().contiguous()
    if qb.dim() != 4 or kb.dim() != 4 or qb.shape[:2] != kb.shape[:2] or qb.shape[3] != kb.shape[3]:
        raise ValueError(f"incompatible block tensors {tuple(qb.shape)} and {tuple(kb.shape)}")
    B, H, nq, D = qb.shape
    nk = kb.shape[2]
    out = torch.empty((B, H, nq, nk), dtype=torch.float32, device=qb.device)
    st = _lib.load().lcv_bsa_scores(qb.data_ptr(), kb.data_ptr(), B, H, nq, nk, D,
                                    out.data_ptr(), _stream(qb))
    _lib.check(st, "block_routing_scores")
    return out


def topk_block_indices(
    score: torch.Tensor, sparsity: float, *, top_k: Optional[int] = None,
) -> tuple[torch.Tensor, int]:
    """Per q-block top-k routing (block_sparse_attention.py:115-134).

    Returns ``(block_indices [B, H, nq, k] int32, k)``; each row lists the
    ``k`` highest-scoring KV blocks in ascending block order.  ``k`` is the
    reference's floor rule unless ``top_k`` is given.
    """
    _require_device(score)
    sc = score.float().contiguous()
    if sc.dim() != 4:
        raise ValueError(f"score must be [B, H, nq, nk], got {tuple(sc.shape)}")
    B, H, nq, nk = sc.shape
    k = num_selected_blocks(nk, sparsity) if top_k is None else int(top_k)
    if not 1 <= k <= nk:
        raise ValueError(f"top_k={k} must be in [1, {nk}]")
    idx = torch.empty((B, H, nq, k), dtype=torch.int32, device=sc.device)
    st = _lib.load().lcv_bsa_topk(sc.data_ptr(), B, H, nq, nk, k, idx.data_ptr(), _stream(sc))
    _lib.check(st, "topk_block_indices")
    return idx, k


def select_block_indices(q_blocks: torch.Tensor, k_blocks: torch.Tensor, top_k: int,
                         *, fused: bool = False) -> torch.Tensor:
    """``topk_block_indices(block_routing_scores(q_blocks, k_blocks))``
    (attention.py:105-108).  By default in two kernels through a transient
    fp32 score tensor (the faster route at 720p sizes); ``fused=True`` runs
    the single kernel that keeps the scores on chip.  At D = 64 or 128 with
    nk <= 2048 both compute every score with the same split-bf16 MFMA
    sequence and give the same selection; elsewhere the fused kernel sums in
    fp32 on the vector ALU, so scores within fp32 rounding of each other may
    be ordered differently."""
    _require_device(q_blocks, k_blocks)
    qb = q_blocks.float().contiguous()
    kb = k_blocks.float().contiguous()
    B, H, nq, D = qb.shape
    nk = kb.shape[2]
    if not 1 <= top_k <= nk:
        raise ValueError(f"top_k={top_k} must be in [1, {nk}]")
    if not fused:
        return topk_block_indices(block_routing_scores(qb, kb), 0.0, top_k=top_k)[0]
    idx = torch.empty((B, H, nq, top_k), dtype=torch.int32, device=qb.device)
    st = _lib.load().lcv_bsa_select(qb.data_ptr(), kb.data_ptr(), B, H, nq, nk, D, top_k,
                                    idx.data_ptr(), _stream(qb))
    _lib.check(st, "select_block_indices")
    return idx


def build_token_block_indices(
    shape: tuple[int, int, int],
    chunk_thw: tuple[int, int, int] = (4, 4, 4),
    device: Optional[torch.device] = None,
) -> torch.Tensor:
    """``[S]`` int32 block id of each t-major token (block_sparse_attention.py:137-159)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    if dev.type != "cuda":
        raise BSADeviceError("the HIP BSA backend builds indices on a ROCm device")
    T, H_, W = shape
    out = torch.empty((T * H_ * W,), dtype=torch.int32, device=dev)
    st = _lib.load().lcv_bsa_token_blocks(_geom(shape, chunk_thw), out.data_ptr(),
                                          torch.cuda.current_stream(dev).cuda_stream)
    _lib.check(st, "build_token_block_indices")
    return out


def build_token_pair_mask(
    block_indices: torch.Tensor,
    token_block_index: torch.Tensor,
    num_kv_blocks: int,
) -> torch.Tensor:
    """``[B, H, S, S]`` bool routing mask (block_sparse_attention.py:162-198).

    Materialises S^2 entries; the attention path never calls it.
    """
    _require_device(block_indices, token_block_index)
    bi = block_indices.to(torch.int32).contiguous()
    tbi = token_block_index.to(torch.int32).contiguous()
    B, H, nq, k = bi.shape
    S = tbi.numel()
    mask = torch.empty((B, H, S, S), dtype=torch.uint8, device=bi.device)
    st = _lib.load().lcv_bsa_token_pair_mask(bi.data_ptr(), B, H, nq, k, tbi.data_ptr(), S,
                                             int(num_kv_blocks), mask.data_ptr(), _stream(bi))
    _lib.check(st, "build_token_pair_mask")
    return mask.view(torch.bool)


def bsa_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    shape: tuple[int, int, int],
    sparsity: float = 0.9375,
    chunk_thw: tuple[int, int, int] = (4, 4, 4),
    sm_scale: Optional[float] = None,
    *,
    top_k: Optional[int] = None,
    return_indices: bool = False,
    block_means: Optional[tuple[torch.Tensor, torch.Tensor]] = None,
    out: Optional[torch.Tensor] = None,
    kv_shape: Optional[tuple[int, int, int]] = None,
):
    """Block Sparse Attention forward (block_sparse_attention.py:201-250).

    q, k, v: ``[B, H, S, D]`` (fp16 / bf16 / fp32) with ``S = T*H*W``;
    ``shape = (T, H, W)`` must be a multiple of ``chunk_thw`` whose product
    is 64.  Returns ``[B, H, S, D]`` in q's dtype, or ``(out, indices)`` with
    ``return_indices=True`` (indices ``[B, H, nb, top_k]`` int32, ascending).
    ``block_means=(q_blocks, k_blocks)`` (fp32 ``[B, H, nb, D]``, e.g. from
    ``prepare_qk``) skips the pooling pass.  ``out`` is an optional
    ``[B, H, S, D]`` destination with unit last stride (e.g. a head-major
    view of a ``[B, S, H, D]`` buffer).

    ``kv_shape`` extends the reference (whose layer sends S_q != S_k to dense
    attention, attention.py:89): k and v are ``[B, H, S_k, D]`` over the
    latent grid ``kv_shape``, cut by the same ``chunk_thw``; each q-block
    keeps the top-k of the ``nk`` k-blocks (the count rule over ``nk``).
    """
    _require_device(q, k, v)
    q, k, v = _bhsd(q, "q"), _bhsd(k, "k"), _bhsd(v, "v")
    if kv_shape is None and not (q.shape == k.shape == v.shape):
        raise ValueError(f"q, k, v shapes differ: {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    B, H, S, D = q.shape
    _check_shape(S, shape, chunk_thw)
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(D)
    nb = num_blocks(shape, chunk_thw)
    nk = nb if kv_shape is None else num_blocks(kv_shape, chunk_thw)
    kk = num_selected_blocks(nk, sparsity) if top_k is None else int(top_k)
    if not 1 <= kk <= nk:
        raise ValueError(f"top_k={kk} must be in [1, {nk}]")
    if block_means is not None or kv_shape is not None:
        from .block_sparse_attention_hip import bsa_attention_hip

        if kv_shape is not None:
            if not (k.shape == v.shape and k.shape[:2] == q.shape[:2] and k.shape[3] == D):
                raise ValueError(f"k, v must be [B, H, S_k, D] matching q {tuple(q.shape)}: "
                                 f"got {tuple(k.shape)}, {tuple(v.shape)}")
            _check_shape(k.shape[2], kv_shape, chunk_thw)
        if block_means is not None:
            qb, kb = block_means
            for name, t, n in (("q_blocks", qb, nb), ("k_blocks", kb, nk)):
                if tuple(t.shape) != (B, H, n, D) or t.dtype != torch.float32:
                    raise ValueError(f"{name} must be fp32 [{B}, {H}, {n}, {D}], got {tuple(t.shape)} {t.dtype}")
        else:
            qb = mean_pool_blocks_3d(q, shape, chunk_thw)
            kb = mean_pool_blocks_3d(k, kv_shape, chunk_thw)
        idx = select_block_indices(qb, kb, kk)
        out = bsa_attention_hip(q, k, v, idx, chunk_thw, shape, sm_scale, out=out, kv_shape=kv_shape)
        return (out, idx) if return_indices else out
    code = _dtype_code(q)
    if code != _lib.F32:
        q, k, v = _aligned_rows(q), _aligned_rows(k), _aligned_rows(v)
    lib = _lib.load()
    from .block_sparse_attention_hip import _output

    out = _output(out, q)
    idx = torch.empty((B, H, nb, kk), dtype=torch.int32, device=q.device)
    ws_bytes = lib.lcv_bsa_forward_workspace_bytes(B, H, nb, D)
    ws = torch.empty((ws_bytes + 255,), dtype=torch.uint8, device=q.device)
    ws_ptr = (ws.data_ptr() + 255) // 256 * 256
    st = lib.lcv_bsa_forward(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), code, B, H, S, D,
        _strides(q), _strides(k), _strides(v), kk, float(sm_scale), _geom(shape, chunk_thw),
        ws_ptr, ws_bytes, idx.data_ptr(), out.data_ptr(), _strides(out), _stream(q),
    )
    _lib.check(st, "bsa_attention")
    return (out, idx) if return_indices else out
