"""Latent-count padding of the 720p refinement pass.

Mirrors ``_compute_padding`` (longcat_video/refinement.py:168-201) and the
config field it reads (``bsa_latent_granularity``, refinement.py:81): before
the VAE encode, the refinement pass pads the conditioning frames at the front
and the noise frames at the back so that both latent counts are multiples of
the BSA voxel's temporal extent (``chunk_3d_shape_q[0]`` = 4).  The latent
grid that reaches ``bsa_attention`` then tiles along time; the spatial axes
are not padded (H_lat = 45 at 720p is handled by the block-geometry policy,
``lcv_bsa.shape_policy``).

Integer arithmetic only: ``-(-a // b)`` is the exact ceiling the reference
takes with ``math.ceil(a / b)`` (identical for every count below 2^53).
"""

from __future__ import annotations

from typing import NamedTuple

__all__ = ["Padding", "compute_padding", "_compute_padding", "DEFAULT_BSA_LATENT_GRANULARITY",
           "DEFAULT_VAE_SCALE_TEMPORAL"]

DEFAULT_VAE_SCALE_TEMPORAL = 4       # RefinementPipelineConfig.vae_scale_temporal (refinement.py:79)
DEFAULT_BSA_LATENT_GRANULARITY = 4   # RefinementPipelineConfig.bsa_latent_granularity (refinement.py:81)


class Padding(NamedTuple):
    """The reference's 4-tuple, by name."""

    num_cond_latents: int
    num_cond_frames_added: int
    num_noise_latents: int
    num_noise_frames_added: int


def _ceil_div(a: int, b: int) -> int:
    return -(-a // b)


def compute_padding(num_cond_frames: int, num_noise_frames: int,
                    vae_scale_temporal: int = DEFAULT_VAE_SCALE_TEMPORAL,
                    bsa_latent_granularity: int = DEFAULT_BSA_LATENT_GRANULARITY) -> Padding:
    """Latent counts and added frames (refinement.py:168-201).

    Conditioning frames (if any) encode causally: the first frame alone,
    then ``vae_scale_temporal`` frames per latent, so ``n`` frames give
    ``1 + ceil((n - 1) / v)`` latents; the count is rounded up to a multiple
    of the granularity and the frames that many latents need,
    ``1 + (latents - 1) * v``, fix how many frames are added (replicated at
    the front by the caller).  Noise frames give ``ceil(n / v)`` latents,
    rounded up the same way, and ``latents * v - n`` frames are added at the
    back.  Returns ``(num_cond_latents, num_cond_frames_added,
    num_noise_latents, num_noise_frames_added)``."""
    v, g = int(vae_scale_temporal), int(bsa_latent_granularity)
    nc, nn = int(num_cond_frames), int(num_noise_frames)
    cond_lat = cond_added = 0
    if nc > 0:
        cond_lat = _ceil_div(1 + _ceil_div(nc - 1, v), g) * g
        cond_added = 1 + (cond_lat - 1) * v - nc
    noise_lat = _ceil_div(_ceil_div(nn, v), g) * g
    noise_added = noise_lat * v - nn
    return Padding(cond_lat, cond_added, noise_lat, noise_added)


# The reference's name for the same rule.
_compute_padding = compute_padding
