"""Seeded synthetic inputs for the BSA forward at the refinement shapes.

Construction (the same for every configuration):

* q, k, v ~ N(0, 1) in fp32;
* q and k get a per-block low-rank offset ``c_b . U`` added to every token
  of block b: ``U`` is a fixed 4 x D matrix with orthonormal rows shared by
  q and k, ``c_b ~ N(0, 0.5^2)`` drawn independently for q and k, per
  (batch, head, block).  This gives the block-score rows clear top-k margins;
* for the refinement shapes, 3D RoPE over the latent grid (T, 45, 80) is
  applied to q and k in fp32 (``lcv_bsa.rope_3d``), then everything is cast
  to the working dtype;
* margin repair: from the cast tensors, fp64 block means and fp64 scores are
  computed, and every (b, h, q-block) row whose gap between the k-th and
  (k+1)-th largest score is <= ``margin`` (for each k in ``margin_ks``) gets
  its q offset re-drawn -- which changes only that score row -- until no row
  is left.  Block selection is then unambiguous for any fp32 evaluation
  order, so indices can be compared exactly.

The BSA geometry of the refinement configurations is contiguous 64-token
blocks, i.e. ``shape=(1, 1, S)``, ``chunk_thw=(1, 1, 64)``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional, Sequence

import torch

from .rope_3d import rope_freqs_3d, apply_rope

__all__ = [
    "CONFIGS", "BSAWorkload", "make_workload", "make_inputs", "block_tokens",
    "executed_flops", "top_k_ceil", "top_k_floor",
]


def top_k_floor(nk: int, sparsity: float) -> int:
    """The reference's rule (block_sparse_attention.py:127)."""
    return max(1, int((1.0 - sparsity) * nk))


def top_k_ceil(nk: int, sparsity: float) -> int:
    """The rule the refinement benchmark shapes are quoted with (29/450, 57/900)."""
    return max(1, math.ceil(round((1.0 - sparsity) * nk, 9)))


def executed_flops(B: int, H: int, nq: int, k: int, D: int, bs: int = 64) -> int:
    """MFMA work on executed blocks: QK^T plus PV, 2 FLOP per MAC."""
    return 4 * B * H * nq * k * bs * bs * D


# name -> parameters.  ``grid`` is the RoPE latent grid (None: no RoPE);
# ``shape``/``chunk`` the BSA geometry.
CONFIGS = {
    # Tier A CPU-runnable case: B1 H2 S4096 D64 fp32, 64 blocks, k=4.
    "c0": dict(B=1, H=2, D=64, dtype=torch.float32, grid=None, shape=(1, 1, 4096),
               chunk=(1, 1, 64), top_k=4),
    # Short clip: 8 x 45 x 80 = 28800 tokens, 450 blocks, k = 29 (ceil) / 28 (floor).
    "c1": dict(B=1, H=32, D=128, dtype=torch.float16, grid=(8, 45, 80), shape=(1, 1, 28800),
               chunk=(1, 1, 64), top_k=29),
    # 720p: 16 x 45 x 80 = 57600 tokens, 900 blocks, k = 57 (ceil) / 56 (floor).
    "c2": dict(B=1, H=32, D=128, dtype=torch.float16, grid=(16, 45, 80), shape=(1, 1, 57600),
               chunk=(1, 1, 64), top_k=57),
    # 720p bf16 CFG batch; the sparsity sweep uses k in {113, 57, 29}.
    "c3": dict(B=2, H=32, D=128, dtype=torch.bfloat16, grid=(16, 45, 80), shape=(1, 1, 57600),
               chunk=(1, 1, 64), top_k=57),
}


@dataclass
class BSAWorkload:
    name: str
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    shape: tuple
    chunk_thw: tuple
    top_k: int
    sm_scale: float
    grid: Optional[tuple]
    seed: int
    repairs: int
    rounds: int
    extra: dict = field(default_factory=dict)

    @property
    def num_blocks(self) -> int:
        return self.q.shape[2] // (self.chunk_thw[0] * self.chunk_thw[1] * self.chunk_thw[2])

    @property
    def flops(self) -> int:
        B, H, _, D = self.q.shape
        return executed_flops(B, H, self.num_blocks, self.top_k, D)


def block_tokens(shape: Sequence[int], chunk: Sequence[int], device=None) -> torch.Tensor:
    """``[nb, bs]`` token index of row r of block n (block-major order)."""
    T, H, W = shape
    cT, cH, cW = chunk
    Bh, Bw = H // cH, W // cW
    nb = (T // cT) * Bh * Bw
    n = torch.arange(nb, device=device)
    bt, bh, bw = n // (Bh * Bw), (n // Bw) % Bh, n % Bw
    r = torch.arange(cT * cH * cW, device=device)
    i, j, l = r // (cH * cW), (r // cW) % cH, r % cW
    base = bt * cT * H * W + bh * cH * W + bw * cW
    return base[:, None] + (i * H * W + j * W + l)[None, :]


def _orthonormal_rows(n: int, D: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed + 7919)
    a = torch.randn(D, n, generator=g, dtype=torch.float64)
    qm, _ = torch.linalg.qr(a)
    return qm.T.contiguous().float()  # (n, D)


def _pooled64(x: torch.Tensor, bt: torch.Tensor, heads_per_chunk: int = 8) -> torch.Tensor:
    """fp64 block means ``[B, H, nb, D]`` of x (any dtype)."""
    B, H, S, D = x.shape
    nb, bs = bt.shape
    out = torch.empty((B, H, nb, D), dtype=torch.float64, device=x.device)
    flat = bt.reshape(-1)
    for b in range(B):
        for h0 in range(0, H, heads_per_chunk):
            xs = x[b, h0:h0 + heads_per_chunk].index_select(1, flat).double()
            out[b, h0:h0 + heads_per_chunk] = xs.view(xs.shape[0], nb, bs, D).mean(dim=2)
    return out


def _bad_rows(qbar: torch.Tensor, kbar: torch.Tensor, ks: Sequence[int], margin: float) -> torch.Tensor:
    score = torch.matmul(qbar, kbar.transpose(-1, -2))  # fp64 [B, H, nq, nk]
    nk = score.shape[-1]
    kmax = min(max(ks) + 1, nk)
    top = torch.topk(score, kmax, dim=-1, sorted=True).values
    bad = torch.zeros(score.shape[:-1], dtype=torch.bool, device=score.device)
    for k in ks:
        if 1 <= k < nk:
            bad |= (top[..., k - 1] - top[..., k]) <= margin
    return bad


def make_inputs(
    B: int, H: int, D: int, shape: Sequence[int], chunk: Sequence[int], dtype: torch.dtype,
    device, seed: int = 0, grid: Optional[Sequence[int]] = None, margin: float = 1e-4,
    margin_ks: Sequence[int] = (), offset_std: float = 0.5, n_dirs: int = 4,
    max_rounds: int = 64,
):
    """Returns ``(q, k, v, info)``; see the module docstring."""
    device = torch.device(device)
    S = int(shape[0]) * int(shape[1]) * int(shape[2])
    bt = block_tokens(shape, chunk, device)
    nb, bs = bt.shape
    gen = torch.Generator(device=device).manual_seed(seed)
    U = _orthonormal_rows(n_dirs, D, seed).to(device)

    def randn(*sz):
        return torch.randn(*sz, generator=gen, device=device, dtype=torch.float32)

    base_q, base_k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
    cq, ck = randn(B, H, nb, n_dirs) * offset_std, randn(B, H, nb, n_dirs) * offset_std
    if grid is not None:
        if int(grid[0]) * int(grid[1]) * int(grid[2]) != S:
            raise ValueError(f"RoPE grid {tuple(grid)} does not cover S={S}")
        f = rope_freqs_3d(tuple(int(x) for x in grid), D, device)
        cos, sin = torch.cos(f), torch.sin(f)
    else:
        cos = sin = None

    def finish(x: torch.Tensor, tok: torch.Tensor) -> torch.Tensor:
        if cos is not None:
            x = apply_rope(x, cos[tok], sin[tok])
        return x.to(dtype)

    def build(base: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
        out = torch.empty((B, H, S, D), dtype=dtype, device=device)
        flat = bt.reshape(-1)
        for b in range(B):
            off = torch.matmul(c[b], U)  # [H, nb, D]
            x = base[b][:, flat].view(H, nb, bs, D) + off[:, :, None, :]
            x = x.view(H, nb * bs, D)
            out[b][:, flat] = finish(x, flat)
        return out

    q = build(base_q, cq)
    k = build(base_k, ck)
    v = v.to(dtype)
    del base_k

    repairs, rounds = 0, 0
    if margin_ks:
        kbar = _pooled64(k, bt)
        qbar = _pooled64(q, bt)
        for rounds in range(1, max_rounds + 1):
            bad = _bad_rows(qbar, kbar, margin_ks, margin)
            nbad = int(bad.sum())
            if nbad == 0:
                break
            repairs += nbad
            bi, hi, ni = bad.nonzero(as_tuple=True)
            cnew = randn(nbad, n_dirs) * offset_std
            cq[bi, hi, ni] = cnew
            tok = bt[ni]  # [nbad, bs]
            rows = base_q[bi[:, None], hi[:, None], tok] + torch.matmul(cnew, U)[:, None, :]
            newq = finish(rows, tok)
            q[bi[:, None], hi[:, None], tok] = newq
            qbar[bi, hi, ni] = newq.double().mean(dim=1)
        else:
            raise RuntimeError(f"margin repair did not converge in {max_rounds} rounds")
    info = dict(repairs=repairs, rounds=rounds, U=U)
    return q, k, v, info


def make_workload(
    name: str, device, seed: int = 0, *, top_k: Optional[int] = None,
    margin_ks: Optional[Sequence[int]] = None, margin: float = 1e-4,
) -> BSAWorkload:
    """One of :data:`CONFIGS`, margin-repaired for its top-k (ceil and floor)."""
    cfg = CONFIGS[name]
    nb = int(cfg["shape"][0] * cfg["shape"][1] * cfg["shape"][2]) // 64
    k = int(top_k if top_k is not None else cfg["top_k"])
    ks = tuple(margin_ks) if margin_ks is not None else tuple(sorted({k, max(1, k - 1)}))
    q, kk, v, info = make_inputs(
        cfg["B"], cfg["H"], cfg["D"], cfg["shape"], cfg["chunk"], cfg["dtype"], device,
        seed=seed, grid=cfg["grid"], margin=margin, margin_ks=ks,
    )
    return BSAWorkload(
        name=name, q=q, k=kk, v=v, shape=tuple(cfg["shape"]), chunk_thw=tuple(cfg["chunk"]),
        top_k=k, sm_scale=1.0 / math.sqrt(cfg["D"]), grid=cfg["grid"], seed=seed,
        repairs=info["repairs"], rounds=info["rounds"], extra={"num_blocks": nb, "margin_ks": ks},
    )
