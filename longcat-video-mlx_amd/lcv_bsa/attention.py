"""BSA dispatch at the attention layer: the ``"hip"`` backend plug-in point.

Mirrors ``Attention._process_attn`` (longcat_video/models/attention.py:71-179):

* BSA runs only when ``enable_bsa`` is set, ``shape`` is given and the query
  and key lengths agree (attention.py:89); otherwise dense attention;
* a ``ValueError`` from the BSA path (shape not a multiple of the voxel,
  unsupported head dim...) falls back to dense attention (attention.py:174-179);
* the dense path uses ``scale = head_dim ** -0.5`` (attention.py:49, 179).

Backends: ``"hip"`` is this package's gfx950 path.  The reference's own
backend names (``"tier_a"``, ``"metal"``, ``"metal_v2"``, ``"metal_v3"``,
``"metal_v4"``; longcat_video_dit.py:249-252) are accepted and run the same
HIP kernels: on the reference they are implementations of one function
(Tier A's masked dense SDPA and the Metal kernels give the same output up to
rounding, bsa.py:201-250, metal.py:75-1046), so an unchanged caller --
``enable_bsa()`` with its default ``"tier_a"``, or scripts/run_refine.py
with ``LONGCAT_BSA_BACKEND`` unset -- gets BSA on MI355X.  The name is kept
on the layer as given; ``resolve_backend`` says which path serves it.
"""

from __future__ import annotations

import os
from typing import Optional

import torch
import torch.nn.functional as F

from .block_sparse_attention import bsa_attention

ENV_VAR = "LONGCAT_BSA_BACKEND"
# The reference's default name (longcat_video_dit.py:219, attention.py:69,
# scripts/run_refine.py:91); it resolves to the HIP path.
DEFAULT_BACKEND = "tier_a"
# Names the reference accepts (longcat_video_dit.py:249), each served here by
# the HIP kernels, plus this package's own name.
REFERENCE_BACKENDS = ("tier_a", "metal", "metal_v2", "metal_v3", "metal_v4")
VALID_BACKENDS = ("hip",) + REFERENCE_BACKENDS

__all__ = [
    "BSAAttention", "ENV_VAR", "DEFAULT_BACKEND", "VALID_BACKENDS", "REFERENCE_BACKENDS",
    "backend_from_env", "validate_backend", "resolve_backend", "dense_attention",
]


def validate_backend(backend: str) -> str:
    """Check a backend name the way longcat_video_dit.py:249-252 does
    (``AssertionError`` for a name outside the accepted set)."""
    assert backend in VALID_BACKENDS, f"unknown BSA backend: {backend!r}. Choose from {VALID_BACKENDS}"
    return backend


def resolve_backend(backend: str) -> str:
    """The implementation that serves ``backend``: ``"hip"`` for every
    accepted name (there is one BSA implementation on MI355X)."""
    validate_backend(backend)
    return "hip"


def backend_from_env(default: str = DEFAULT_BACKEND) -> str:
    """``LONGCAT_BSA_BACKEND`` as read by scripts/run_refine.py:91-92
    (unset -> ``"tier_a"``, as there)."""
    return os.environ.get(ENV_VAR, default)


def dense_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """Dense SDPA, the dispatcher's fallback (attention.py:179).

    On the GPU only torch's fused SDPA kernels are used, never its math path
    (its batched products take a transposed bf16 operand); where no fused
    kernel applies, the scores are formed in fp32 over row chunks with
    contiguous operands.  On the CPU, plain SDPA."""
    if q.device.type != "cuda":
        return F.scaled_dot_product_attention(q, k, v, scale=scale)
    from torch.nn.attention import SDPBackend, sdpa_kernel

    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, scale=scale)
    except RuntimeError:
        pass
    kt = k.float().transpose(-1, -2).contiguous()
    vf = v.float().contiguous()
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    step = 4096
    for s0 in range(0, q.shape[-2], step):
        s = torch.matmul(q[..., s0:s0 + step, :].float().contiguous(), kt) * scale
        out[..., s0:s0 + step, :] = torch.matmul(torch.softmax(s, dim=-1), vf).to(q.dtype)
    return out


class BSAAttention:
    """The BSA-relevant state of the reference ``Attention`` layer.

    Holds the four attributes ``enable_bsa`` / ``bsa_sparsity`` /
    ``bsa_chunk_thw`` / ``bsa_backend`` that ``enable_bsa()`` sets on every
    block (dit.py:253-257; attention.py:62-69) plus ``head_dim``/``scale``,
    and implements ``_process_attn``.  A PyTorch port of the LongCat
    ``Attention`` module can inherit from it unchanged.
    """

    def __init__(self, dim: int, num_heads: int):
        assert dim % num_heads == 0, "dim must be divisible by num_heads"
        self.dim = dim
        self.num_heads = num_heads
        self.head_dim = dim // num_heads
        self.scale = self.head_dim ** -0.5
        self.enable_bsa: bool = False
        self.bsa_sparsity: float = 0.9375
        self.bsa_chunk_thw: tuple[int, int, int] = (4, 4, 4)
        self.bsa_backend: str = DEFAULT_BACKEND
        # Optional explicit block count (overrides the sparsity rule).
        self.bsa_top_k: Optional[int] = None
        # Filled by each call: "bsa" or "dense" (for callers and tests).
        self.last_path: str = ""

    def _process_attn(
        self,
        q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
        shape: Optional[tuple[int, int, int]] = None,
    ) -> torch.Tensor:
        """q, k, v: ``[B, H, S, D]``; returns ``[B, H, S_q, D]``."""
        if self.enable_bsa and shape is not None and q.shape[-2] == k.shape[-2]:
            resolve_backend(self.bsa_backend)  # every accepted name runs the HIP kernels
            try:
                out = bsa_attention(
                    q, k, v, shape=shape,
                    sparsity=self.bsa_sparsity,
                    chunk_thw=self.bsa_chunk_thw,
                    sm_scale=self.scale,
                    top_k=self.bsa_top_k,
                )
                self.last_path = "bsa"
                return out
            except ValueError:
                # Shape not a multiple of the voxel (or a configuration the
                # kernels do not cover): dense, as the reference does.
                pass
        self.last_path = "dense"
        return dense_attention(q, k, v, self.scale)
