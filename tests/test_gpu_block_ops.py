"""GPU parity of the DiT block's fused row operations (lcv_bsa_block_rows,
lcv_bsa_block_swiglu, lcv_bsa_head_rms_norm) against the oracle.

The residual r = round(x + gate * a) is pure fp32 arithmetic and must match
an fp32 NumPy restatement bit for bit.  The normalised outputs may differ in
the summation order of the LayerNorm statistics (and exp in the gate), so
they must equal the oracle on almost every element and stay within one unit
in the last place of the dtype everywhere.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import bsa_oracle as O
from oracle import dit_block_oracle as DB

pytestmark = pytest.mark.gpu

NAME = {torch.float16: "f16", torch.bfloat16: "bf16"}
ULP = {torch.float16: 2.0 ** -10, torch.bfloat16: 2.0 ** -7}


def _np(t):
    return t.detach().float().cpu().numpy()


def _rand(shape, dtype, device, seed, scale=1.0, shift=0.0):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale + shift).to(dtype).to(device)


def _close_ulp(got, ref, dtype, what, exact_frac=0.99, floor=2.0 ** -6, ulps=1):
    """Within ``ulps`` units in the last place of |ref| (at least ``floor``:
    near zero, fp32 differences in the row statistics -- e.g. the mean of
    4096 values summed in another order -- are larger than the dtype's
    spacing)."""
    ulp = ulps * ULP[dtype] * np.maximum(np.abs(ref), floor)
    err = np.abs(got - ref)
    assert np.all(err <= ulp * 1.01), f"{what}: max {np.max(err / ulp):.2f} ulp"
    assert np.mean(err == 0) >= exact_frac, f"{what}: only {np.mean(err == 0):.4f} exact"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("C", [256, 4096])
def test_residual_norm_modes_match_oracle(device, dtype, C):
    from lcv_bsa.block_ops import residual_norm

    B, T, per = 2, 3, 64
    N = T * per
    x = _rand((B, N, C), dtype, device, 1, 2.0, 0.5)
    a = _rand((B, N, C), dtype, device, 2)
    g = torch.Generator(device="cpu").manual_seed(3)
    gate, shift, scale = (torch.randn(B, T, 1, C, generator=g).to(device) * s for s in (0.7, 0.3, 0.2))
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(dtype).to(device)
    bias = (0.1 * torch.randn(C, generator=g)).to(dtype).to(device)
    nm = NAME[dtype]
    xs, as_, gs, shs, scs = _np(x), _np(a), _np(gate), _np(shift), _np(scale)

    # Gated residual (fp32 ops, rounded): bit-exact.
    ref_r = O.round_to((xs.reshape(B, T, per, C) + gs.astype(np.float32) * as_.reshape(B, T, per, C))
                       .reshape(B, N, C).astype(np.float32), nm)
    r, n = residual_norm(x, a, gate, frames=T, weight=w, bias=bias)
    assert np.array_equal(_np(r), ref_r), "gated residual"
    ref_n = O.round_to(DB.layer_norm_fp32(ref_r, _np(w), _np(bias)), nm)
    _close_ulp(_np(n), ref_n, dtype, f"affine LN C={C}")

    # Plain residual + AdaLN modulation.
    r2, m2 = residual_norm(x, a, frames=T, shift=shift, scale=scale)
    ref_r2 = O.round_to(xs + as_, nm)
    assert np.array_equal(_np(r2), ref_r2), "plain residual"
    ref_m2 = DB.modulate_fp32(ref_r2.reshape(B, T, per, C), shs, scs, nm).reshape(B, N, C)
    _close_ulp(_np(m2), ref_m2, dtype, f"modulation C={C}")

    # Modulation only; gated residual only.
    _, m = residual_norm(x, frames=T, shift=shift, scale=scale)
    _close_ulp(_np(m), DB.modulate_fp32(xs.reshape(B, T, per, C), shs, scs, nm).reshape(B, N, C), dtype,
               "modulate only")
    r4, none = residual_norm(x, a, gate, frames=T, norm=False)
    assert none is None and torch.equal(r4, r)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_swiglu_matches_oracle(device, dtype):
    from lcv_bsa.block_ops import swiglu

    h = _rand((3, 70, 2 * 264), dtype, device, 5, 3.0)
    out = swiglu(h)
    hs = _np(h)
    a, b = hs[..., :264], hs[..., 264:]
    s = O.round_to(DB.silu(a).astype(np.float32), NAME[dtype])
    ref = O.round_to(s * b, NAME[dtype])
    assert out.shape == (3, 70, 264)
    _close_ulp(_np(out), ref, dtype, "swiglu", exact_frac=0.98)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128])
def test_head_rms_norm_matches_oracle(device, dtype, D):
    from lcv_bsa.block_ops import head_rms_norm

    B, N, H = 2, 96, 3
    x = _rand((B, N, H, D), dtype, device, 7, 1.5, 0.2)
    w = (1 + 0.2 * torch.randn(D, generator=torch.Generator().manual_seed(8))).to(dtype).to(device)
    ref = O.rms_norm_fp32(np.transpose(_np(x), (0, 2, 1, 3)), _np(w), 1e-6, NAME[dtype])
    out = head_rms_norm(x.transpose(1, 2), w)                 # strided in, contiguous [B, H, N, D] out
    assert out.is_contiguous()
    # One ulp for rsqrt's rounding of the normalised value (which the weight
    # multiply carries through) plus one for the final rounding.
    _close_ulp(_np(out), ref, dtype, f"head norm D={D}", exact_frac=0.99, ulps=2)
    y = x.clone()
    head_rms_norm(y.transpose(1, 2), w, out=y.transpose(1, 2))  # in place
    assert torch.equal(y.transpose(1, 2), out)


def test_block_ops_reject_bad_arguments(device):
    from lcv_bsa.block_ops import residual_norm, swiglu

    x = _rand((1, 128, 256), torch.bfloat16, device, 9)
    with pytest.raises(ValueError):
        residual_norm(x, frames=3)                       # 128 tokens do not split into 3 frames
    with pytest.raises(ValueError):
        residual_norm(x.float(), frames=2)
    with pytest.raises(ValueError):
        swiglu(_rand((4, 2 * 12), torch.bfloat16, device, 10))   # hidden 12 is not a multiple of 8


@pytest.mark.parametrize("fused", [True, False])
def test_block_fused_and_unfused_paths_agree_with_oracle(device, fused):
    """The same block through the fused row kernels / fused cross-attention /
    fused SwiGLU, and through the torch ops, against the oracle."""
    from lcv_bsa.dit_block import LongCatSingleStreamBlock
    from lcv_bsa.shape_policy import bsa_geometry

    C, H, t_dim, L, grid = 256, 2, 64, 64, (4, 8, 16)
    N = int(np.prod(grid))
    torch.manual_seed(0)
    blk = LongCatSingleStreamBlock(C, H, 4, t_dim, dtype=torch.bfloat16, device=device)
    g = torch.Generator(device="cpu").manual_seed(0)
    with torch.no_grad():
        for name, p in blk.named_parameters():
            if name.endswith("norm.weight") or name == "pre_crs_attn_norm.weight":
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(0.05 * torch.randn(p.shape, generator=g))
    for m in (blk, blk.ffn, blk.cross_attn):
        m.fused = fused
    a = blk.attn
    a.enable_bsa, a.bsa_chunk_thw, a.bsa_top_k, a.keep_indices = True, (4, 4, 4), 3, True
    x = _rand((1, N, C), torch.bfloat16, device, 11)
    y = _rand((1, L, C), torch.bfloat16, device, 12)
    t = torch.randn(1, grid[0], t_dim, generator=torch.Generator().manual_seed(13)).to(device)
    with torch.no_grad():
        out = blk(x, y, t, [L], grid)
    p = {k: _np(v) for k, v in blk.state_dict().items()}
    idx = {k: v.cpu().numpy() for k, v in a.last_indices.items()}
    ref, _ = DB.dit_block(_np(x), _np(y), _np(t), p, grid, H, "bf16",
                          {"all": bsa_geometry(grid, (4, 4, 4), "reference"), "top_k": 3}, idx)
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    err = np.abs(_np(out).astype(np.float64) - ref)
    bound = 2 * 2.0 ** -8 * np.abs(ref) + 0.02 * rms
    assert np.all(err <= bound), f"fused={fused}: max excess {np.max(err / bound):.2f}"
    assert err.mean() < 0.005 * rms
