"""BSA dispatch at the attention layer: the ``"hip"`` backend plug-in point.

Mirrors ``Attention._process_attn`` (longcat_video/models/attention.py:71-179):

* BSA runs only when ``enable_bsa`` is set, ``shape`` is given and the query
  and key lengths agree (attention.py:89); otherwise dense attention;
* a ``ValueError`` from the BSA path (shape not a multiple of the voxel,
  unsupported head dim...) falls back to dense attention (attention.py:174-179);
* the dense path uses ``scale = head_dim ** -0.5`` (attention.py:49, 179).

Backends: ``"hip"`` is this package's gfx950 path.  The reference's own
backend names (``tier_a``, ``metal*``) need MLX on Apple hardware and are
rejected with a clear error rather than silently remapped.
"""

from __future__ import annotations

import os
from typing import Optional

import torch
import torch.nn.functional as F

from .block_sparse_attention import bsa_attention

ENV_VAR = "LONGCAT_BSA_BACKEND"
DEFAULT_BACKEND = "hip"
VALID_BACKENDS = ("hip",)
REFERENCE_ONLY_BACKENDS = ("tier_a", "metal", "metal_v2", "metal_v3", "metal_v4")

__all__ = [
    "BSAAttention", "ENV_VAR", "DEFAULT_BACKEND", "VALID_BACKENDS", "REFERENCE_ONLY_BACKENDS",
    "backend_from_env", "validate_backend", "dense_attention",
]


def validate_backend(backend: str) -> str:
    """Check a backend name the way dit.py:249-252 does (AssertionError)."""
    assert backend in VALID_BACKENDS, (
        f"unknown BSA backend: {backend!r}. Choose from {VALID_BACKENDS}"
        + (" (the reference's MLX/Metal backends do not exist on MI355X)"
           if backend in REFERENCE_ONLY_BACKENDS else "")
    )
    return backend


def backend_from_env(default: str = DEFAULT_BACKEND) -> str:
    """``LONGCAT_BSA_BACKEND`` as read by scripts/run_refine.py:91-92."""
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
            validate_backend(self.bsa_backend)
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
