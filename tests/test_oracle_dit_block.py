"""Pins the DiT-block oracle (oracle/dit_block_oracle.py) before the torch +
HIP block is compared against it.

Checks are the reference's known answer for the SwiGLU width
(tests/smoke/test_blocks_smoke.py:29-38), closed forms (LayerNorm moments,
silu values, attention over one key or identical keys), reductions to pieces
pinned elsewhere (BSA with every block selected is dense attention; the
oracle's dense attention is torch's CPU SDPA), the AdaLN-zero identity of the
block, and planted mistakes that those checks must catch.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle import bsa_oracle as O
from oracle import dit_block_oracle as DB

RNG = np.random.default_rng(77)


def _params(C, H, mlp_ratio=4, t_dim=32, scale=0.05, seed=0):
    rng = np.random.default_rng(seed)
    p = {}
    for name, shp in DB.block_param_shapes(C, H, mlp_ratio, t_dim).items():
        if name.endswith("norm.weight") or name == "pre_crs_attn_norm.weight":
            p[name] = (1.0 + 0.1 * rng.normal(size=shp)).astype(np.float32)
        else:
            p[name] = (scale * rng.normal(size=shp)).astype(np.float32)
    return p


def test_swiglu_width_known_answer():
    # test_blocks_smoke.py:29-38: dim 4096, hidden 4*4096, multiple_of 256 -> 11008.
    assert DB.swiglu_hidden_dim(4 * 4096) == 11008
    assert DB.swiglu_hidden_dim(256, 16) == 176          # int(512/3) = 170 -> 176
    assert DB.swiglu_hidden_dim(4 * 128) == 512          # 341 -> 512
    assert DB.block_param_shapes(4096, 32)["ffn.w2.weight"] == (4096, 11008)


def test_silu_closed_forms():
    assert DB.silu(0.0) == 0.0
    assert math.isclose(DB.silu(1.0), 1.0 / (1.0 + math.exp(-1.0)), rel_tol=1e-15)
    assert math.isclose(DB.silu(30.0), 30.0, rel_tol=1e-12)
    assert abs(DB.silu(-30.0)) < 1e-11
    x = RNG.normal(size=100)
    assert np.allclose(DB.silu(x), torch.nn.functional.silu(torch.from_numpy(x)).numpy(), rtol=1e-12)


def test_layer_norm_known_answer_and_moments():
    y = DB.layer_norm_fp32(np.array([[1.0, 2.0, 3.0, 4.0]]), eps=0.0)
    assert np.allclose(y, (np.array([1, 2, 3, 4]) - 2.5) / math.sqrt(1.25), rtol=1e-6)
    x = RNG.normal(size=(16, 256)) * 3 + 5
    y = DB.layer_norm_fp32(x, eps=1e-6).astype(np.float64)
    assert np.allclose(y.mean(-1), 0.0, atol=1e-6) and np.allclose(y.var(-1), 1.0, atol=1e-4)
    w, b = RNG.normal(size=256), RNG.normal(size=256)
    assert np.allclose(DB.layer_norm_fp32(x, w, b), y * w + b, atol=1e-5)
    t = torch.nn.functional.layer_norm(torch.from_numpy(x), (256,), torch.from_numpy(w), torch.from_numpy(b), 1e-6)
    assert np.allclose(DB.layer_norm_fp32(x, w, b), t.numpy(), atol=1e-5)


def test_planted_sample_variance_is_caught():
    x = RNG.normal(size=(4, 8))
    m = x.mean(-1, keepdims=True)
    planted = (x - m) / np.sqrt(x.var(-1, ddof=1, keepdims=True) + 1e-6)
    assert not np.allclose(planted, DB.layer_norm_fp32(x), atol=1e-3)


def test_modulate_scale_plus_one_and_per_frame_broadcast():
    x = RNG.normal(size=(1, 3, 5, 16)).astype(np.float32)
    zero = np.zeros((1, 3, 1, 16), np.float32)
    assert np.array_equal(DB.modulate_fp32(x, zero, zero, "f32"), DB.layer_norm_fp32(x))
    shift = zero.copy()
    shift[0, 1] = 2.0                                    # frame 1 only
    scale = np.full((1, 3, 1, 16), 0.5, np.float32)
    y = DB.modulate_fp32(x, shift, scale, "f32")
    ln = DB.layer_norm_fp32(x)
    assert np.allclose(y[0, 0], 1.5 * ln[0, 0], atol=1e-6)
    assert np.allclose(y[0, 1], 1.5 * ln[0, 1] + 2.0, atol=1e-6)
    planted = ln * scale + shift                         # scale instead of scale + 1
    assert not np.allclose(planted, y, atol=1e-3)


def test_feed_forward_identity_weights_closed_form():
    x = RNG.normal(size=(1, 4, 8)).astype(np.float32)
    eye = np.eye(8, dtype=np.float32)
    y = DB.feed_forward_swiglu(x, eye, eye, eye, "f32")
    assert np.allclose(y, DB.silu(x) * x, rtol=1e-6, atol=1e-7)
    # w1 and w3 play different roles: swapping them must change the output.
    w1, w3 = RNG.normal(size=(8, 8)).astype(np.float32), RNG.normal(size=(8, 8)).astype(np.float32)
    a = DB.feed_forward_swiglu(x, w1, eye, w3, "f32")
    b = DB.feed_forward_swiglu(x, w3, eye, w1, "f32")
    assert not np.allclose(a, b)


def test_dense_attention_closed_forms_and_torch():
    q = RNG.normal(size=(1, 2, 5, 8))
    v1 = RNG.normal(size=(1, 2, 1, 8))
    assert np.allclose(DB.dense_attention(q, RNG.normal(size=(1, 2, 1, 8)), v1, 0.3), np.broadcast_to(v1, q.shape))
    k_same = np.broadcast_to(RNG.normal(size=(1, 2, 1, 8)), (1, 2, 6, 8))
    v = RNG.normal(size=(1, 2, 6, 8))
    assert np.allclose(DB.dense_attention(q, k_same, v, 0.3), np.broadcast_to(v.mean(2, keepdims=True), q.shape))
    k = RNG.normal(size=(1, 2, 6, 8))
    t = torch.nn.functional.scaled_dot_product_attention(*(torch.from_numpy(a) for a in (q, k, v)), scale=0.3)
    assert np.allclose(DB.dense_attention(q, k, v, 0.3), t.numpy(), atol=1e-12)


def test_self_attention_with_all_blocks_is_dense():
    """BSA with every KV block selected reduces to dense attention, so the
    layer must equal qkv -> RMSNorm -> RoPE -> dense attention -> proj."""
    C, H, grid = 128, 2, (2, 8, 16)
    p = _params(C, H)
    N = int(np.prod(grid))
    x = O.round_to(RNG.normal(size=(1, N, C)).astype(np.float32), "bf16")
    bsa = {"all": ((1, 1, N), (1, 1, 64)), "top_k": N // 64}
    out, idx = DB.self_attention(x, p, grid, H, "bf16", bsa)
    idx = idx["all"]
    assert np.array_equal(np.sort(idx, -1), np.broadcast_to(np.arange(N // 64), idx.shape))
    # Dense path through the oracle's own (pinned) pieces.
    D = C // H
    qkv = DB.linear(x, p["attn.qkv.weight"], p["attn.qkv.bias"], "bf16").reshape(1, N, 3, H, D)
    q, k, v = (np.transpose(qkv[:, :, i], (0, 2, 1, 3)) for i in range(3))
    q = O.rms_norm_fp32(q, p["attn.q_norm.weight"], 1e-6, "bf16")
    k = O.rms_norm_fp32(k, p["attn.k_norm.weight"], 1e-6, "bf16")
    f = O.rope_freqs_3d(grid, D).astype(np.float32)
    q = O.round_to(O.apply_rope(q, f), "bf16")
    k = O.round_to(O.apply_rope(k, f), "bf16")
    o = O.round_to(O.sdpa(q, k, v, D ** -0.5).astype(np.float32), "bf16")
    ref = DB.linear(np.transpose(o, (0, 2, 1, 3)).reshape(1, N, C), p["attn.proj.weight"], p["attn.proj.bias"], "bf16")
    assert np.allclose(out, ref, atol=2e-2, rtol=2e-2)
    assert np.mean(out == ref) > 0.9


def test_cross_attention_closed_forms():
    C, H = 128, 2
    p = _params(C, H)
    x = RNG.normal(size=(1, 7, C)).astype(np.float32)
    # One text token: every query reads the same v row, so all rows are equal.
    y1 = RNG.normal(size=(1, 1, C)).astype(np.float32)
    out = DB.cross_attention(x, y1, p, H, "f32")
    assert np.allclose(out, np.broadcast_to(out[:, :1], out.shape), atol=1e-6)
    kv = DB.linear(y1, p["cross_attn.kv_linear.weight"], p["cross_attn.kv_linear.bias"], "f32")
    v = kv.reshape(1, 1, 2, C)[:, :, 1]
    assert np.allclose(out[0, 0], DB.linear(v, p["cross_attn.proj.weight"], p["cross_attn.proj.bias"], "f32")[0, 0],
                       atol=1e-5)
    # Zero output projection: the bias alone.
    p0 = dict(p)
    p0["cross_attn.proj.weight"] = np.zeros_like(p["cross_attn.proj.weight"])
    y = RNG.normal(size=(1, 9, C)).astype(np.float32)
    assert np.allclose(DB.cross_attention(x, y, p0, H, "f32"),
                       np.broadcast_to(p["cross_attn.proj.bias"], (1, 7, C)), atol=1e-7)


def test_block_adaln_zero_identity_and_planted_gate():
    """AdaLN-zero: with zero modulation (so zero gates) and a zero cross-attn
    projection the block returns x exactly."""
    C, H, grid = 128, 2, (2, 8, 16)
    N = int(np.prod(grid))
    p = _params(C, H)
    for name in ("adaLN_modulation.1.weight", "adaLN_modulation.1.bias", "cross_attn.proj.weight",
                 "cross_attn.proj.bias"):
        p[name] = np.zeros_like(p[name])
    x = O.round_to(RNG.normal(size=(1, N, C)).astype(np.float32), "bf16")
    y = RNG.normal(size=(1, 5, C)).astype(np.float32)
    t = RNG.normal(size=(1, grid[0], 32)).astype(np.float32)
    bsa = {"all": ((1, 1, N), (1, 1, 64)), "top_k": 2}
    out, _ = DB.dit_block(x, y, t, p, grid, H, "bf16", bsa)
    assert np.array_equal(out, x)
    # A gate of one on the attention branch of frame 1 only changes frame 1's tokens.
    p["adaLN_modulation.1.bias"] = np.zeros(6 * C, np.float32)
    p["adaLN_modulation.1.weight"] = np.zeros((6 * C, 32), np.float32)
    p["adaLN_modulation.1.weight"][2 * C:3 * C, 0] = 1.0          # gate_msa = silu(t[..., 0])
    t2 = np.zeros_like(t)
    t2[0, 1, 0] = 5.0
    out2, _ = DB.dit_block(x, y, t2, p, grid, H, "bf16", bsa)
    per = N // grid[0]
    assert np.array_equal(out2[:, :per], x[:, :per])
    assert not np.array_equal(out2[:, per:], x[:, per:])


def _qkv_roped(x, p, grid, H, dtype="bf16"):
    N, C = x.shape[1], x.shape[2]
    D = C // H
    qkv = DB.linear(x, p["attn.qkv.weight"], p["attn.qkv.bias"], dtype).reshape(1, N, 3, H, D)
    q, k, v = (np.transpose(qkv[:, :, i], (0, 2, 1, 3)) for i in range(3))
    q = O.rms_norm_fp32(q, p["attn.q_norm.weight"], 1e-6, dtype)
    k = O.rms_norm_fp32(k, p["attn.k_norm.weight"], 1e-6, dtype)
    f = O.rope_freqs_3d(grid, D).astype(np.float32)
    return O.round_to(O.apply_rope(q, f), dtype), O.round_to(O.apply_rope(k, f), dtype), v


def test_cond_split_with_all_blocks_is_masked_dense():
    """attention.py:202-221 with every block selected: conditioning queries
    see only conditioning keys, noise queries see all keys -- one dense
    attention (torch's SDPA) under that mask."""
    C, H, grid, ncl = 128, 2, (4, 8, 8), 2
    N = int(np.prod(grid))
    nc = N // grid[0] * ncl
    p = _params(C, H, seed=3)
    x = O.round_to(RNG.normal(size=(1, N, C)).astype(np.float32), "bf16")
    bsa = {"cond": ((1, 1, nc), (1, 1, 64)), "noise": (((1, 1, N - nc), (1, 1, 64)), ((1, 1, N), (1, 1, 64))),
           "top_k": 1}
    every = {"cond": np.broadcast_to(np.arange(nc // 64), (1, H, nc // 64, nc // 64)),
             "noise": np.broadcast_to(np.arange(N // 64), (1, H, (N - nc) // 64, N // 64))}
    out_all, _ = DB.self_attention(x, p, grid, H, "bf16", bsa, block_indices=every, num_cond_latents=ncl)
    q, k, v = _qkv_roped(x, p, grid, H)
    mask = np.zeros((N, N))
    mask[:nc, nc:] = -np.inf
    o = torch.nn.functional.scaled_dot_product_attention(*(torch.from_numpy(a.astype(np.float64)) for a in (q, k, v)),
                                                         attn_mask=torch.from_numpy(mask), scale=(C // H) ** -0.5)
    o = O.round_to(o.numpy().astype(np.float32), "bf16")
    ref = DB.linear(np.transpose(o, (0, 2, 1, 3)).reshape(1, N, C), p["attn.proj.weight"], p["attn.proj.bias"], "bf16")
    assert np.allclose(out_all, ref, atol=2e-2, rtol=2e-2) and np.mean(out_all == ref) > 0.9
    # The split is not the unsplit layer: conditioning rows differ from full attention.
    full, _ = DB.self_attention(x, p, grid, H, "bf16", {"all": None, "top_k": 1})
    assert not np.allclose(full[:, :nc], out_all[:, :nc], atol=1e-3)
    assert np.allclose(full[:, nc:], out_all[:, nc:], atol=2e-2)


def test_kv_cache_continuation_equals_split_noise_branch():
    """attention.py:235-275: continuing from the cache of the conditioning
    frames gives the noise rows of the conditioning split, when the chunk's
    tokens are the noise frames (RoPE over the extended grid aligns them)."""
    C, H, full_grid, ncl = 128, 2, (4, 8, 8), 2
    N = int(np.prod(full_grid))
    nc = N // full_grid[0] * ncl
    p = _params(C, H, seed=4)
    x = O.round_to(RNG.normal(size=(1, N, C)).astype(np.float32), "bf16")
    dense = {"cond": None, "noise": None, "top_k": 1}
    split, _ = DB.self_attention(x, p, full_grid, H, "bf16", dense, num_cond_latents=ncl)
    # The cache: normed, un-rotated k / v of the conditioning frames.
    D = C // H
    qkv = DB.linear(x[:, :nc], p["attn.qkv.weight"], p["attn.qkv.bias"], "bf16").reshape(1, nc, 3, H, D)
    kc = O.rms_norm_fp32(np.transpose(qkv[:, :, 1], (0, 2, 1, 3)), p["attn.k_norm.weight"], 1e-6, "bf16")
    vc = np.transpose(qkv[:, :, 2], (0, 2, 1, 3))
    noise_grid = (full_grid[0] - ncl,) + full_grid[1:]
    cont, _ = DB.self_attention_kv_cache(x[:, nc:], p, noise_grid, H, "bf16", (kc, vc), ncl, dense)
    assert np.array_equal(cont, split[:, nc:])


def _block_check(got, ref, dtype_ulp, what):
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    err = np.abs(got.astype(np.float64) - ref)
    bound = 2 * dtype_ulp * np.abs(ref) + 0.02 * rms
    assert np.all(err <= bound), f"{what}: max excess {np.max(err / bound):.2f}"
    assert err.mean() < 0.005 * rms, f"{what}: mean error {err.mean() / rms:.2e} of rms"
    return float(np.max(err / bound))


def test_torch_block_reference_matches_oracle():
    """The torch fp32 restatement used at 720p on the GPU (tests/block_reference.py)
    agrees with the NumPy block oracle on a small block in fp16 and bf16,
    with BSA routed over 64-token runs, and a planted dropped FFN gate is
    caught."""
    from block_reference import dit_block_torch

    C, H, t_dim, L, grid, top_k = 128, 2, 32, 16, (4, 4, 16), 2
    N = int(np.prod(grid))
    p = _params(C, H, t_dim=t_dim, seed=5)
    rng = np.random.default_rng(6)
    for dt, name, ulp in ((torch.float16, "f16", 2.0 ** -11), (torch.bfloat16, "bf16", 2.0 ** -8)):
        x = O.round_to(rng.normal(size=(1, N, C)).astype(np.float32), name)
        y = O.round_to(rng.normal(size=(1, L, C)).astype(np.float32), name)
        t = rng.normal(size=(1, grid[0], t_dim)).astype(np.float32)
        idx = np.sort(np.stack([rng.choice(N // 64, size=top_k, replace=False)
                                for _ in range(H * (N // 64))]), -1).reshape(1, H, N // 64, top_k)
        idx = idx.astype(np.int32)
        ref, _ = DB.dit_block(x, y, t, p, grid, H, name, {"all": ((1, 1, N), (1, 1, 64)), "top_k": top_k},
                              block_indices={"all": idx})
        tp = {k: torch.from_numpy(v) for k, v in p.items()}
        args = (torch.from_numpy(x).to(dt), torch.from_numpy(y).to(dt), torch.from_numpy(t))
        got = dit_block_torch(*args, tp, grid, H, dt, torch.from_numpy(idx)).numpy()
        _block_check(got, ref, ulp, f"torch block reference {name}")
        tp_bad = dict(tp)
        tp_bad["ffn.w2.weight"] = torch.zeros_like(tp["ffn.w2.weight"])
        bad = dit_block_torch(*args, tp_bad, grid, H, dt, torch.from_numpy(idx)).numpy()
        assert np.abs(bad - ref).max() > 0.1
