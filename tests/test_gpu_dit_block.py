"""GPU parity of one DiT block (torch GEMMs + the HIP attention path) against
the NumPy block oracle (oracle/dit_block_oracle.py, itself pinned by
tests/test_oracle_dit_block.py).

The oracle takes the GPU run's block routing (``attn.last_indices``): the
routing itself is checked bit-exactly against the oracle's top-k elsewhere,
and near-tied block scores computed from bf16 values may legitimately pick a
different block.  Everything else -- modulation, fused RMSNorm + RoPE, BSA,
cross-attention, SwiGLU, gated residuals -- is compared with a model-dtype
tolerance: each element within two ulps of the oracle (fp16: 2^-10, bf16:
2^-7 relative) plus 2 % of the output's rms, and a mean error under 0.5 % of
the rms.

The full 720p block (hidden 4096, 32 heads, 16 x 45 x 80 latents, 512 text
tokens) runs in fp16 -- the activation dtype of the benchmark's block config
-- and in bf16 with every branch live (random AdaLN modulation and
projections), against tests/block_reference.py (the oracle restated in fp32
torch, pinned against it on the CPU).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import dit_block_oracle as DB

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy()


ULP = {torch.float16: 2.0 ** -11, torch.bfloat16: 2.0 ** -8}
ORACLE_DTYPE = {torch.float16: "f16", torch.bfloat16: "bf16"}


def _block(C, H, t_dim, device, seed=0, std=0.05, dtype=torch.bfloat16):
    from lcv_bsa.dit_block import LongCatSingleStreamBlock

    torch.manual_seed(seed)
    blk = LongCatSingleStreamBlock(C, H, 4, t_dim, dtype=dtype, device=device)
    g = torch.Generator(device="cpu").manual_seed(seed)
    with torch.no_grad():
        for name, p in blk.named_parameters():
            if name.endswith("norm.weight") or name == "pre_crs_attn_norm.weight":
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(std * torch.randn(p.shape, generator=g))
    return blk


def _inputs(N, C, T, t_dim, L, device, seed=1, dtype=torch.bfloat16):
    g = torch.Generator(device="cpu").manual_seed(seed)
    x = torch.randn(1, N, C, generator=g).to(dtype).to(device)
    y = torch.randn(1, L, C, generator=g).to(dtype).to(device)
    t = torch.randn(1, T, t_dim, generator=g).to(device)
    return x, y, t


def _check(got, ref, what, ulp=2.0 ** -8):
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    err = np.abs(got.astype(np.float64) - ref)
    bound = 2 * ulp * np.abs(ref) + 0.02 * rms
    assert np.all(err <= bound), f"{what}: max excess {np.max(err / bound):.2f}"
    assert err.mean() < 0.005 * rms, f"{what}: mean error {err.mean() / rms:.2e} of rms"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("policy,grid,chunk", [
    ("reference", (4, 8, 16), (4, 4, 4)),
    ("auto", (4, 6, 16), (4, 4, 4)),          # voxel does not tile H=6: contiguous 64-token blocks
])
def test_block_matches_oracle(device, policy, grid, chunk, dtype):
    C, H, t_dim, L = 256, 2, 64, 24
    N = int(np.prod(grid))
    blk = _block(C, H, t_dim, device, dtype=dtype)
    blk.attn.enable_bsa, blk.attn.bsa_chunk_thw, blk.attn.bsa_shape_policy = True, chunk, policy
    blk.attn.bsa_top_k, blk.attn.keep_indices = 3, True
    x, y, t = _inputs(N, C, grid[0], t_dim, L, device, dtype=dtype)
    with torch.no_grad():
        out = blk(x, y, t, [L], grid)
    assert blk.attn.last_path == "bsa"
    idx = blk.attn.last_indices["all"].cpu().numpy()
    from lcv_bsa.shape_policy import bsa_geometry

    p = {k: _np(v) for k, v in blk.state_dict().items()}
    ref, _ = DB.dit_block(_np(x), _np(y), _np(t), p, grid, H, ORACLE_DTYPE[dtype],
                          {"all": bsa_geometry(grid, chunk, policy), "top_k": 3}, block_indices={"all": idx})
    _check(_np(out), ref, f"block {policy} {grid} {dtype}", ULP[dtype])
    assert idx.shape == (1, H, N // 64, 3) and np.all(np.diff(idx, axis=-1) > 0)


def test_block_reference_policy_falls_back_to_dense(device):
    """The reference policy with a voxel that does not tile the grid runs
    dense attention (attention.py:174-179), and the block still matches."""
    C, H, t_dim, L, grid = 256, 2, 64, 16, (4, 6, 16)
    N = int(np.prod(grid))
    blk = _block(C, H, t_dim, device, seed=3)
    blk.attn.enable_bsa, blk.attn.bsa_chunk_thw = True, (4, 4, 4)
    x, y, t = _inputs(N, C, grid[0], t_dim, L, device, seed=4)
    with torch.no_grad():
        out = blk(x, y, t, [L], grid)
    assert blk.attn.last_path == "dense"
    p = {k: _np(v) for k, v in blk.state_dict().items()}
    nb = N // 64
    ref, _ = DB.dit_block(_np(x), _np(y), _np(t), p, grid, H, "bf16", {"all": None, "top_k": nb})
    _check(_np(out), ref, "dense fallback")


def test_bsa_out_view_matches_default(device):
    """bsa_attention(out=<[B,S,H,D] buffer>.transpose(1, 2)) writes the same
    bits as the default contiguous output."""
    from lcv_bsa import bsa_attention

    g = torch.Generator(device="cpu").manual_seed(9)
    B, H, S, D = 1, 4, 2048, 128
    q, k, v = (torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).to(device) for _ in range(3))
    ref = bsa_attention(q, k, v, (1, 1, S), chunk_thw=(1, 1, 64), top_k=5)
    buf = torch.full((B, S, H, D), float("nan"), dtype=torch.bfloat16, device=device)
    got = bsa_attention(q, k, v, (1, 1, S), chunk_thw=(1, 1, 64), top_k=5, out=buf.transpose(1, 2))
    assert got.data_ptr() == buf.data_ptr()
    assert torch.equal(buf.transpose(1, 2), ref)


def test_block_720p_adaln_zero_is_identity(device):
    """Full 720p block (hidden 4096, 32 heads, 16 x 45 x 80 latents, 512 text
    tokens) on the BSA path: with zero AdaLN modulation and a zero
    cross-attention projection every branch is gated off, so the block
    returns x bit for bit, whatever the branches computed."""
    from lcv_bsa.dit_block import LongCatSingleStreamBlock

    grid = (16, 45, 80)
    N = int(np.prod(grid))
    blk = LongCatSingleStreamBlock(4096, 32, 4, 512, dtype=torch.bfloat16, device=device)
    with torch.no_grad():
        for p in blk.parameters():
            p.normal_(0.0, 0.02)
        for p in (blk.adaLN_modulation[1].weight, blk.adaLN_modulation[1].bias,
                  blk.cross_attn.proj.weight, blk.cross_attn.proj.bias):
            p.zero_()
    blk.attn.enable_bsa, blk.attn.bsa_shape_policy, blk.attn.bsa_top_k = True, "auto", 57
    x, y, t = _inputs(N, 4096, grid[0], 512, 512, device, seed=5)
    with torch.no_grad():
        out = blk(x, y, t, [512], grid)
    torch.cuda.synchronize()
    assert blk.attn.last_path == "bsa"
    assert torch.equal(out, x)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_block_720p_matches_torch_reference(device, dtype):
    """One DiT block at the benchmark's config (720p latents 16 x 45 x 80 =
    57,600 tokens, hidden 4096, 32 heads x 128, SwiGLU 11008, 512 text
    tokens, random weights and AdaLN, top-k 57 of 900 64-token blocks) with
    every branch live, against the oracle restated in fp32 torch
    (tests/block_reference.py) on the same routing."""
    from block_reference import dit_block_torch

    torch.backends.cuda.matmul.allow_tf32 = False
    grid, C, H, L, t_dim = (16, 45, 80), 4096, 32, 512, 512
    N = int(np.prod(grid))
    print(f"720p block {dtype}: building", flush=True)
    blk = _block(C, H, t_dim, device, seed=21, std=0.02, dtype=dtype)
    blk.attn.enable_bsa, blk.attn.bsa_shape_policy, blk.attn.bsa_top_k = True, "auto", 57
    blk.attn.keep_indices = True
    x, y, t = _inputs(N, C, grid[0], t_dim, L, device, seed=22, dtype=dtype)
    with torch.no_grad():
        out = blk(x, y, t, [L], grid)
        torch.cuda.synchronize()
        assert blk.attn.last_path == "bsa"
        idx = blk.attn.last_indices["all"]
        assert idx.shape == (1, H, N // 64, 57)
        lin = blk.adaLN_modulation[1]
        ada = torch.nn.functional.linear(torch.nn.functional.silu(t.float()), lin.weight.float(), lin.bias.float())
        gate_rms = float(ada.pow(2).mean().sqrt())
        assert gate_rms > 0.05, "modulation too small to exercise the branches"
        print(f"720p block {dtype}: HIP block done, reference next", flush=True)
        p = {k: v.detach() for k, v in blk.state_dict().items()}
        ref, env = dit_block_torch(x, y, t, p, grid, H, dtype, idx, envelope=True)
        torch.cuda.synchronize()
        # the branches moved x: the check is not of the identity
        moved = float((out.float() - x.float()).abs().mean())
        assert moved > 1e-2, f"block output equals its input (mean change {moved:.2e})"
        # Bounds in units of the model dtype's ulp (relative 2^-11 for fp16,
        # 2^-8 for bf16), the same for both dtypes: each element within 4 ulps
        # of the magnitudes summed into it plus 10 ulps of the output's rms,
        # and the mean error within 1 ulp of the rms.  Both sides round the
        # same terms at the same points; GEMMs that accumulate in other orders
        # flip single roundings of q / k / intermediate activations, which the
        # attention logits and the FFN carry to every element (the measured
        # maximum is ~6 ulps of the rms and the mean ~0.4 ulp, in either dtype).
        err = (out.float() - ref).abs()
        rms = float(ref.pow(2).mean().sqrt())
        ulp = ULP[dtype]
        excess = float((err / (4 * ulp * env + 10 * ulp * rms)).max())
        max_ulp_rms = float(err.max()) / (ulp * rms)
        mean_ulp_rms = float(err.mean()) / (ulp * rms)
    print(f"720p block {dtype}: rms {rms:.3f}, max err {float(err.max()):.3e} = {max_ulp_rms:.2f} ulp*rms, "
          f"mean err {mean_ulp_rms:.3f} ulp*rms, worst err / bound {excess:.3f}, mean change {moved:.3f}", flush=True)
    assert excess <= 1.0, f"720p block {dtype}: an element exceeds its bound by {excess:.2f}x"
    assert mean_ulp_rms <= 1.0, f"720p block {dtype}: mean error {mean_ulp_rms:.2f} ulp of the rms"


# ---------------------------------------------------------------------------
# Conditioning split and KV-cache continuation (S_q != S_k on the noise side)
# ---------------------------------------------------------------------------

def _attn_params(blk):
    return {"attn." + k: _np(v) for k, v in blk.attn.state_dict().items()}


def _split_geoms(grid, ncl, chunk, policy, cond_noise, top_k):
    from lcv_bsa.shape_policy import bsa_geometry

    T, Hl, Wl = grid
    cond, noise = (ncl, Hl, Wl), (T - ncl, Hl, Wl)
    return {"cond": bsa_geometry(cond, chunk, policy),
            "noise": (bsa_geometry(noise, chunk, policy), bsa_geometry(grid, chunk, policy)) if cond_noise else None,
            "top_k": top_k}


def _idx(blk):
    return {k: v.cpu().numpy() for k, v in blk.attn.last_indices.items()}


@pytest.mark.parametrize("policy,chunk,cond_noise", [
    ("reference", (4, 4, 4), False),      # the reference: cond via BSA, noise dense
    ("reference", (4, 4, 4), True),       # noise queries over all keys via BSA (kv geometry)
    ("contiguous", (4, 4, 4), True),
])
def test_attention_cond_split_matches_oracle(device, policy, chunk, cond_noise):
    C, H, grid, ncl = 256, 2, (8, 8, 16), 4
    N = int(np.prod(grid))
    blk = _block(C, H, 64, device, seed=7)
    a = blk.attn
    a.enable_bsa, a.bsa_chunk_thw, a.bsa_shape_policy = True, chunk, policy
    a.bsa_cond_noise, a.bsa_top_k, a.keep_indices = cond_noise, 3, True
    x, _, _ = _inputs(N, C, grid[0], 64, 8, device, seed=8)
    with torch.no_grad():
        out = a(x, grid, ncl)
    assert a.last_paths == {"cond": "bsa", "noise": "bsa" if cond_noise else "dense"}
    idx = _idx(blk)
    ref, _ = DB.self_attention(_np(x), _attn_params(blk), grid, H, "bf16",
                               _split_geoms(grid, ncl, chunk, policy, cond_noise, 3), idx, ncl)
    _check(_np(out), ref, f"cond split {policy} cond_noise={cond_noise}")


@pytest.mark.parametrize("cond_noise", [False, True])
def test_attention_kv_cache_matches_oracle(device, cond_noise):
    """Cache the conditioning frames (return_kv), then continue the noise
    frames from it (attention.py:235-275)."""
    C, H, grid, ncl = 256, 2, (8, 8, 16), 4
    N = int(np.prod(grid))
    nc = N // grid[0] * ncl
    noise_grid = (grid[0] - ncl,) + grid[1:]
    blk = _block(C, H, 64, device, seed=9)
    a = blk.attn
    a.enable_bsa, a.bsa_chunk_thw, a.bsa_cond_noise, a.bsa_top_k, a.keep_indices = True, (4, 4, 4), cond_noise, 3, True
    x, _, _ = _inputs(N, C, grid[0], 64, 8, device, seed=10)
    with torch.no_grad():
        _, (kc, vc) = a(x[:, :nc], (ncl,) + grid[1:], return_kv=True)
        out = a.forward_with_kv_cache(x[:, nc:], noise_grid, ncl, (kc, vc))
    assert a.last_paths["noise"] == ("bsa" if cond_noise else "dense")
    bsa = _split_geoms(grid, ncl, (4, 4, 4), "reference", cond_noise, 3)
    ref, _ = DB.self_attention_kv_cache(_np(x[:, nc:]), _attn_params(blk), noise_grid, H, "bf16",
                                        (_np(kc), _np(vc)), ncl, bsa, _idx(blk))
    _check(_np(out), ref, f"kv cache cond_noise={cond_noise}")


def test_block_with_cond_latents_matches_oracle(device):
    C, H, t_dim, L, grid, ncl = 256, 2, 64, 16, (8, 8, 16), 4
    N = int(np.prod(grid))
    blk = _block(C, H, t_dim, device, seed=11)
    a = blk.attn
    a.enable_bsa, a.bsa_chunk_thw, a.bsa_cond_noise, a.bsa_top_k, a.keep_indices = True, (4, 4, 4), True, 3, True
    x, y, t = _inputs(N, C, grid[0], t_dim, L, device, seed=12)
    with torch.no_grad():
        out = blk(x, y, t, [L], grid, num_cond_latents=ncl)
    p = {k: _np(v) for k, v in blk.state_dict().items()}
    ref, _ = DB.dit_block(_np(x), _np(y), _np(t), p, grid, H, "bf16",
                          _split_geoms(grid, ncl, (4, 4, 4), "reference", True, 3), _idx(blk), num_cond_latents=ncl)
    _check(_np(out), ref, "block with cond latents")
