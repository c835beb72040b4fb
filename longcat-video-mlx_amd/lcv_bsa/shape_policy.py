"""Which block geometry BSA uses for a latent grid.

The reference calls BSA with the latent shape and ``bsa_chunk_thw``
(attention.py:89-173); when the voxel does not tile the grid,
``mean_pool_blocks_3d`` raises ``ValueError`` (block_sparse_attention.py:
86-90) and the layer silently runs dense attention (attention.py:174-179).
At 720p the latent grid is (T, 45, 80), and 45 rows are not a multiple of the
default (4, 4, 4) voxel, so the refinement pass never uses BSA there.

Policies:

* ``"reference"``: the reference's behaviour -- (shape, chunk_thw) as given,
  dense when the voxel does not tile the grid;
* ``"contiguous"``: blocks of 64 consecutive tokens in the t-major order,
  i.e. ``shape=(1, 1, S)``, ``chunk_thw=(1, 1, 64)`` (needs S % 64 == 0);
* ``"auto"``: the given voxel when it tiles the grid, else contiguous blocks,
  else dense.

Contiguous blocks are runs of 64 tokens along W (80 wide at 720p), so a block
spans at most two latent rows of one frame: spatially compact, but flatter
than a 4 x 4 x 4 voxel.  Padding H to 48 instead would add 6.7 % more tokens
whose keys the attention would have to exclude, and which the reference's
kernels have no mask for; it is not offered.
"""

from __future__ import annotations

from typing import Optional, Sequence

__all__ = ["POLICIES", "bsa_geometry"]

POLICIES = ("reference", "contiguous", "auto")


def _tiles(shape: Sequence[int], chunk: Sequence[int]) -> bool:
    return all(int(s) % int(c) == 0 for s, c in zip(shape, chunk))


def bsa_geometry(
    latent_shape: Sequence[int], chunk_thw: Sequence[int], policy: str = "reference"
) -> Optional[tuple[tuple[int, int, int], tuple[int, int, int]]]:
    """(shape, chunk_thw) to hand to BSA for ``latent_shape``, or ``None`` for
    dense attention.  ``"reference"`` returns the inputs unchanged (BSA then
    raises ``ValueError`` exactly where the reference does)."""
    if policy not in POLICIES:
        raise ValueError(f"unknown BSA shape policy {policy!r}; choose from {POLICIES}")
    shape = tuple(int(x) for x in latent_shape)
    chunk = tuple(int(x) for x in chunk_thw)
    S = shape[0] * shape[1] * shape[2]
    contiguous = ((1, 1, S), (1, 1, 64)) if S % 64 == 0 else None
    if policy == "reference":
        return shape, chunk
    if policy == "contiguous":
        return contiguous
    if _tiles(shape, chunk) and chunk[0] * chunk[1] * chunk[2] == 64:
        return shape, chunk
    return contiguous
