"""End-to-end parity of the HIP ``bsa_attention`` with the oracle's Tier A.

Mirrors tests/smoke/test_bsa_tier_a_smoke.py on the device, checks the
routing bit-exactly (as ascending sets) on margin-repaired inputs, and the
output within the fp16 tolerance of the north-star contract
(max-abs 2e-3, mean-abs 2e-4 against fp64) -- bf16 / fp32 as in
test_gpu_kernels.py.  Also covers the ``_process_attn`` dispatcher.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from conftest import assert_close_report
from oracle import bsa_oracle as O

pytestmark = pytest.mark.gpu

TOL = {torch.float16: (2e-3, 2e-4), torch.bfloat16: (1e-2, 2e-3), torch.float32: (2e-5, 2e-6)}


def _np(t):
    return t.detach().float().cpu().numpy()


def test_sparsity_zero_equals_dense(device):
    """test_bsa_tier_a_smoke.py:141-162 (fp32, < 1e-4)."""
    from lcv_bsa import bsa_attention

    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 4, 64, 16, generator=g).to(device) for _ in range(3))
    out = bsa_attention(q, k, v, shape=(4, 4, 4), sparsity=0.0)
    dense = torch.nn.functional.scaled_dot_product_attention(q.cpu(), k.cpu(), v.cpu(), scale=0.25)
    assert float((out.cpu() - dense).abs().max()) < 1e-4


def test_realistic_shape_finite(device):
    """test_bsa_tier_a_smoke.py:165-184."""
    from lcv_bsa import bsa_attention

    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 2, 256, 32, generator=g).to(device) for _ in range(3))
    out = bsa_attention(q, k, v, shape=(4, 8, 8), sparsity=0.9375)
    assert out.shape == (1, 2, 256, 32) and torch.isfinite(out).all()


def test_rejects_non_multiple_shape(device):
    """test_bsa_tier_a_smoke.py:187-196."""
    from lcv_bsa import bsa_attention

    q = torch.zeros((1, 1, 96, 8), device=device)
    with pytest.raises(ValueError, match="multiple of"):
        bsa_attention(q, q, q, shape=(4, 4, 6), sparsity=0.9)


CASES = [
    # name, B, H, D, dtype, bsa shape, chunk, rope grid, top_k (None = floor rule)
    ("c0", 1, 2, 64, torch.float32, (1, 1, 4096), (1, 1, 64), None, 4),
    ("voxel444", 1, 2, 128, torch.float16, (8, 16, 16), (4, 4, 4), (8, 16, 16), None),
    ("rope_fp16", 1, 4, 128, torch.float16, (1, 1, 2048), (1, 1, 64), (2, 16, 64), 3),
    ("rope_bf16", 2, 2, 128, torch.bfloat16, (1, 1, 2048), (1, 1, 64), (2, 16, 64), 5),
    ("d64_fp16", 1, 3, 64, torch.float16, (4, 8, 32), (4, 4, 4), None, 7),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_bsa_matches_tier_a(device, case):
    from lcv_bsa import bsa_attention
    from lcv_bsa.workloads import make_inputs

    name, B, H, D, dtype, shape, chunk, grid, top_k = case
    nb = int(np.prod(shape)) // 64
    k_eff = O.num_selected(nb, 0.9375) if top_k is None else top_k
    q, k, v, info = make_inputs(B, H, D, shape, chunk, dtype, device, seed=sum(map(ord, name)),
                                grid=grid, margin_ks=(k_eff,))
    print(f"{name}: margin repairs={info['repairs']}")
    out, idx = bsa_attention(q, k, v, shape=shape, chunk_thw=chunk, top_k=top_k,
                             return_indices=True)
    qn, kn, vn = _np(q), _np(k), _np(v)
    ref, ref_idx = O.bsa_attention(qn, kn, vn, shape, 0.9375, chunk, top_k=top_k,
                                   return_indices=True)
    assert np.array_equal(idx.cpu().numpy(), ref_idx), f"{name}: routing differs"
    assert out.dtype == dtype
    assert_close_report(_np(out), ref, *TOL[dtype], name)
    if int(np.prod(shape)) <= 4096 and B * H <= 4:
        masked = O.bsa_attention_masked(qn, kn, vn, shape, 0.9375, chunk, top_k=top_k)
        assert_close_report(_np(out), masked, *TOL[dtype], name + " (masked form)")


def test_golden_c0(device):
    """The committed C0 fixture: routing exact, output within fp32 tolerance."""
    from pathlib import Path

    from lcv_bsa import bsa_attention
    from lcv_bsa.workloads import make_workload

    fx = np.load(Path(__file__).parent / "golden" / "c0.npz")
    w = make_workload("c0", "cpu", seed=int(fx["seed"]))
    assert np.isclose(float(w.q.double().sum()), float(fx["q_sum"]), rtol=0, atol=1e-6)
    q, k, v = (t.to(device) for t in (w.q, w.k, w.v))
    out, idx = bsa_attention(q, k, v, shape=w.shape, chunk_thw=w.chunk_thw, top_k=w.top_k,
                             return_indices=True)
    assert np.array_equal(idx.cpu().numpy(), fx["indices"])
    rows = fx["rows"]
    assert_close_report(_np(out)[:, :, rows], fx["out_rows"], *TOL[torch.float32], "golden c0")


# ---------------------------------------------------------------------------
# Dispatcher (attention.py:71-179) with the "hip" backend
# ---------------------------------------------------------------------------

def test_process_attn_routes_to_hip(device):
    from lcv_bsa import BSAAttention, bsa_attention
    from lcv_bsa.workloads import make_inputs

    attn = BSAAttention(dim=4 * 128, num_heads=4)
    attn.enable_bsa = True
    attn.bsa_chunk_thw = (4, 4, 4)
    q, k, v, _ = make_inputs(1, 4, 128, (8, 8, 16), (4, 4, 4), torch.float16, device, seed=3)
    out = attn._process_attn(q, k, v, shape=(8, 8, 16))
    assert attn.last_path == "bsa"
    ref = bsa_attention(q, k, v, shape=(8, 8, 16), chunk_thw=(4, 4, 4), sm_scale=128 ** -0.5)
    assert torch.equal(out, ref)


def test_process_attn_dense_fallbacks(device):
    from lcv_bsa import BSAAttention

    attn = BSAAttention(dim=2 * 64, num_heads=2)
    attn.enable_bsa = True
    g = torch.Generator().manual_seed(1)
    q, k, v = (torch.randn(1, 2, 96, 64, generator=g).to(device) for _ in range(3))
    dense = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=64 ** -0.5)
    # 4x4x6 is not a multiple of the voxel -> ValueError -> dense (attention.py:174-179)
    out = attn._process_attn(q, k, v, shape=(4, 4, 6))
    assert attn.last_path == "dense" and torch.allclose(out, dense)
    # shape None -> dense (attention.py:89)
    out = attn._process_attn(q, k, v, shape=None)
    assert attn.last_path == "dense"
    # S_q != S_k -> dense
    out = attn._process_attn(q[:, :, :64], k, v, shape=(4, 4, 4))
    assert attn.last_path == "dense" and out.shape == (1, 2, 64, 64)


def test_env_backend_selection(device, monkeypatch):
    from lcv_bsa.dit import enable_bsa_from_env

    class Blk:
        def __init__(self):
            from lcv_bsa import BSAAttention
            self.attn = BSAAttention(256, 2)

    class Model:
        blocks = [Blk(), Blk()]

    monkeypatch.setenv("LONGCAT_BSA_BACKEND", "hip")
    assert enable_bsa_from_env(Model) == "hip"
    assert all(b.attn.enable_bsa and b.attn.bsa_backend == "hip" for b in Model.blocks)


@pytest.mark.parametrize("name", ["tier_a", "metal", "metal_v4"])
def test_reference_backend_names_run_bsa(device, monkeypatch, name):
    """An unchanged refinement setup: LONGCAT_BSA_BACKEND unset (-> "tier_a",
    scripts/run_refine.py:91) or a Metal name runs BSA through the HIP
    kernels, with the same bits as the "hip" name."""
    from lcv_bsa import BSAAttention
    from lcv_bsa.dit import enable_bsa_from_env
    from lcv_bsa.workloads import make_inputs

    class Blk:
        def __init__(self):
            self.attn = BSAAttention(4 * 128, 4)

    class Model:
        blocks = [Blk()]

    if name == "tier_a":
        monkeypatch.delenv("LONGCAT_BSA_BACKEND", raising=False)
    else:
        monkeypatch.setenv("LONGCAT_BSA_BACKEND", name)
    assert enable_bsa_from_env(Model) == name
    attn = Model.blocks[0].attn
    q, k, v, _ = make_inputs(1, 4, 128, (8, 8, 16), (4, 4, 4), torch.float16, device, seed=5)
    out = attn._process_attn(q, k, v, shape=(8, 8, 16))
    assert attn.last_path == "bsa"
    attn.bsa_backend = "hip"
    assert torch.equal(out, attn._process_attn(q, k, v, shape=(8, 8, 16)))


def test_golden_voxel(device):
    """The committed (4,4,4)-voxel fp16 fixture, end to end."""
    from pathlib import Path

    from lcv_bsa import bsa_attention

    fx = np.load(Path(__file__).parent / "golden" / "voxel.npz")
    shape, chunk = tuple(int(x) for x in fx["shape"]), tuple(int(x) for x in fx["chunk"])
    q, k, v = (torch.from_numpy(fx[n]).to(device) for n in ("q", "k", "v"))
    out, idx = bsa_attention(q, k, v, shape=shape, sparsity=float(fx["sparsity"]), chunk_thw=chunk,
                             return_indices=True)
    assert np.array_equal(idx.cpu().numpy(), fx["indices"])
    assert_close_report(_np(out), fx["out"], *TOL[torch.float16], "golden voxel")
