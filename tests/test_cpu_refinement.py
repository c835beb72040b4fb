"""The refinement pass's latent padding rule (longcat_video/refinement.py:168-201).

Pinned by the reference's own known answers (tests/smoke/test_refinement_smoke.py:
67-91) and, over a grid of frame counts, VAE strides and granularities, by a
brute-force search that restates what the rule must achieve: the smallest
latent count that is a multiple of the granularity and whose frames cover the
input (causal VAE for conditioning frames, plain stride for noise frames).
"""

from __future__ import annotations

import itertools

import pytest

from lcv_bsa.refinement import Padding, _compute_padding, compute_padding


def test_known_answers_from_reference_smoke():
    # 23 noise frames: ceil(23/4) = 6 latents -> 8; 8*4 - 23 = 9 frames added.
    assert compute_padding(num_cond_frames=0, num_noise_frames=23, vae_scale_temporal=4,
                           bsa_latent_granularity=4) == (0, 0, 8, 9)
    # 8 conditioning frames: 1 + ceil(7/4) = 3 latents -> 4; 1 + 3*4 - 8 = 5 frames added.
    nc_lat, nc_added, nn_lat, nn_added = compute_padding(8, 10, 4, 4)
    assert (nc_lat, nc_added) == (4, 5)
    assert (nn_lat, nn_added) == (4, 6)
    assert _compute_padding is compute_padding


def _cond_brute(n: int, v: int, g: int) -> tuple[int, int]:
    if n <= 0:
        return 0, 0
    L = g
    while 1 + (L - 1) * v < n:  # a causal VAE turns 1 + (L - 1) v frames into L latents
        L += g
    return L, 1 + (L - 1) * v - n


def _noise_brute(n: int, v: int, g: int) -> tuple[int, int]:
    L = 0
    while L * v < n:
        L += g
    return L, L * v - n


@pytest.mark.parametrize("v,g", list(itertools.product((1, 2, 4, 8), (1, 2, 4, 8))))
def test_matches_brute_force(v, g):
    for nc in range(0, 70):
        for nn in range(0, 130):
            got = compute_padding(nc, nn, v, g)
            assert isinstance(got, Padding)
            assert (got.num_cond_latents, got.num_cond_frames_added) == _cond_brute(nc, v, g), (nc, v, g)
            assert (got.num_noise_latents, got.num_noise_frames_added) == _noise_brute(nn, v, g), (nn, v, g)
            assert got.num_cond_latents % g == 0 and got.num_noise_latents % g == 0
            assert got.num_cond_frames_added >= 0 and got.num_noise_frames_added >= 0


def test_720p_refinement_grid():
    """The 720p refinement latents of the benchmark (16 frames of 45 x 80):
    61..64 noise frames pad to 64 and give 16 latents, a multiple of the
    (4, 4, 4) voxel's temporal extent; 65 frames need the next multiple."""
    for n in range(61, 65):
        assert compute_padding(0, n) == (0, 0, 16, 64 - n)
    assert compute_padding(0, 65) == (0, 0, 20, 15)
    # a continuation with 13 conditioning frames: 1 + ceil(12/4) = 4 latents, no padding
    assert compute_padding(13, 64)[:2] == (4, 0)
    assert compute_padding(14, 64)[:2] == (8, 15)
