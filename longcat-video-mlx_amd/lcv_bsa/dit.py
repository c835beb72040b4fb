"""Model-level BSA switches: ``from_config`` parameters, ``enable_bsa`` /
``disable_bsa`` (longcat_video/models/longcat_video_dit.py:193-262).

Works on any model object whose ``blocks`` each carry an ``attn`` with the
:class:`~lcv_bsa.attention.BSAAttention` attributes, so a PyTorch port of the
LongCat DiT gets the reference's switches by mixing in :class:`BSAModelMixin`.
"""

from __future__ import annotations

from typing import Any, Mapping

from .attention import DEFAULT_BACKEND, backend_from_env, validate_backend

__all__ = ["BSAModelMixin", "apply_bsa_params", "enable_bsa", "disable_bsa", "enable_bsa_from_env"]


def apply_bsa_params(model: Any, config: Mapping[str, Any]) -> None:
    """Keep the published ``bsa_params`` on the model (dit.py:208-217) and
    honour ``enable_bsa`` from the config (published default: false)."""
    bsa_params = config.get("bsa_params") or {}
    model._bsa_sparsity = float(bsa_params.get("sparsity", 0.9375))
    model._bsa_chunk_thw = tuple(bsa_params.get("chunk_3d_shape_q", [4, 4, 4]))
    if config.get("enable_bsa", False):
        enable_bsa(model)


def enable_bsa(model: Any, backend: str = DEFAULT_BACKEND) -> None:
    """Turn BSA on in every block (dit.py:220-257)."""
    validate_backend(backend)
    sparsity = getattr(model, "_bsa_sparsity", 0.9375)
    chunk = tuple(getattr(model, "_bsa_chunk_thw", (4, 4, 4)))
    for block in model.blocks:
        block.attn.enable_bsa = True
        block.attn.bsa_sparsity = sparsity
        block.attn.bsa_chunk_thw = chunk
        block.attn.bsa_backend = backend


def disable_bsa(model: Any) -> None:
    """Turn BSA off in every block (dit.py:259-262)."""
    for block in model.blocks:
        block.attn.enable_bsa = False


def enable_bsa_from_env(model: Any) -> str:
    """``dit.enable_bsa(backend=os.environ.get("LONGCAT_BSA_BACKEND", ...))``
    as scripts/run_refine.py:86-94 does; returns the backend used."""
    backend = backend_from_env()
    enable_bsa(model, backend)
    return backend


class BSAModelMixin:
    """Adds the reference's ``enable_bsa`` / ``disable_bsa`` methods."""

    _bsa_sparsity: float = 0.9375
    _bsa_chunk_thw: tuple = (4, 4, 4)

    def enable_bsa(self, backend: str = DEFAULT_BACKEND) -> None:
        enable_bsa(self, backend)

    def disable_bsa(self) -> None:
        disable_bsa(self)
