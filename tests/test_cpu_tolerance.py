"""Pins the bf16 bound of the wide-score-range attention tests on the CPU.

At bf16 and D = 64 those tests allow 2e-2 max-abs instead of the general
1e-2.  The reason is the output format, not the kernel: some outputs reach
|o| >= 4, where a bf16 ulp is 2^-5, so even the correctly rounded bf16 of the
exact result misses the fp64 oracle by up to 2^-6 (1.3-1.4e-2 on the q-scale
inputs).  These tests compute that
floor, and an ideal kernel (exact row maxima, P rounded once to bf16, sums in
fp64, output rounded to bf16), on the very inputs of the GPU tests.

A wrong emulation fails here: leaving out the output rounding gives about
3.4e-3, below the asserted floor of the q-scale inputs; leaving out the P
rounding makes the P-only error vanish, outside its asserted (1e-3, 5e-3).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from conftest import wide_range_inputs
from oracle import bsa_oracle as O

SHAPE, CHUNK = (1, 1, 2048), (1, 1, 64)


def _bf16(x: torch.Tensor) -> torch.Tensor:
    return x.float().to(torch.bfloat16).double()


def _emulate(q, k, v, idx):
    """fp64 attention over the listed keys (every q-block lists the same
    blocks in these inputs), returning (exact, P rounded, ideal kernel)."""
    D = q.shape[-1]
    blocks = np.sort(idx[0, 0, 0])
    assert (np.sort(idx, axis=-1) == blocks).all()
    keys = np.concatenate([np.arange(64 * b, 64 * b + 64) for b in blocks])
    q64, k64, v64 = (t.double() for t in (q, k, v))
    s = torch.matmul(q64, k64[:, :, keys].transpose(-1, -2)) / np.sqrt(D)
    p = torch.exp(s - s.max(-1, keepdim=True).values)
    exact = torch.matmul(p, v64[:, :, keys]) / p.sum(-1, keepdim=True)
    pb = _bf16(p)
    p_rounded = torch.matmul(pb, v64[:, :, keys]) / pb.sum(-1, keepdim=True)
    return exact, p_rounded, _bf16(p_rounded)


CASES = [dict(q_scale=s) for s in (1.0, 6.0, 12.0)] + [
    dict(q_scale=12.0, seeds=(41, 42, 43), wide_rows=r) for r in ((0, 32), (32, 64), (16, 48))]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{v}" for v in c.values()))
def test_bf16_wide_range_floor(case):
    q, k, v, idx = wide_range_inputs(64, dtype=torch.bfloat16, **case)
    ref = O.sparse_attention_from_indices(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          idx, SHAPE, CHUNK)
    exact, p_rounded, ideal = _emulate(q, k, v, idx)
    # The emulation's exact path is the oracle.
    assert np.abs(exact.numpy() - ref).max() < 1e-12
    # Floor: the correctly rounded output, at most half an ulp of the largest
    # output (in [4, 8) here: 2^-6).
    floor = np.abs(_bf16(exact).numpy() - ref).max()
    big = np.abs(ref).max()
    assert 4.0 <= big < 8.0
    assert floor <= 2.0 ** -6
    if "wide_rows" not in case:
        # The inputs on which the GPU test needs the wider bound: no kernel
        # that returns bf16 can meet 1e-2 on them.
        assert floor > 1e-2, f"correctly rounded bf16 misses by only {floor:.3e}"
    # The ideal kernel: that floor plus the P rounding, within 2e-2.
    p_only = np.abs(p_rounded.numpy() - ref).max()
    err = np.abs(ideal.numpy() - ref).max()
    assert 1e-3 < p_only < 5e-3
    assert floor - 1e-3 <= err <= 2e-2
    print(f"{case}: max|ref| {big:.2f}  floor {floor:.3e}  P rounding {p_only:.3e}  ideal {err:.3e}")


@pytest.mark.parametrize("q_scale", [1.0, 6.0, 12.0])
def test_bf16_wide_range_d128_within_general_bound(q_scale):
    """At D = 128 the same construction leaves the ideal kernel inside the
    general bf16 bound of 1e-2, which those GPU cases keep."""
    q, k, v, idx = wide_range_inputs(128, q_scale, torch.bfloat16)
    ref = O.sparse_attention_from_indices(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                          idx, SHAPE, CHUNK)
    _, _, ideal = _emulate(q, k, v, idx)
    assert np.abs(ideal.numpy() - ref).max() <= 1e-2
