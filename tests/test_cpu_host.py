"""CPU tests of the host side: the C-ABI library loads and exports what
include/lcv_bsa.h declares, its argument validation (paths that return before
any launch), the dispatcher / enable_bsa wiring (mirroring
tests/smoke/test_bsa_dit_wiring_smoke.py) and the workload generator."""

from __future__ import annotations

import math
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import bsa_oracle as O

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "lcv_bsa.h"
NO_GPU = not torch.cuda.is_available()


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const char\*|int|int64_t|size_t)\s+(lcv_bsa_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    from lcv_bsa import _lib

    assert _declared() == sorted(_lib.EXPORTED)


def test_library_loads_and_exports_every_symbol():
    import ctypes

    from lcv_bsa import _lib

    lib = _lib.load()
    for name in _declared():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name
    assert "gfx950" in _lib.version()
    for code in range(7):
        assert lib.lcv_bsa_strerror(code)
    assert lib.lcv_bsa_strerror(99) == b"unknown status"


@pytest.mark.skipif(not NO_GPU, reason="validation-only calls use fake pointers; CPU container only")
def test_c_abi_validation_returns_before_launch():
    """Each call below must be rejected by argument checks (no launch)."""
    from lcv_bsa import _lib

    lib = _lib.load()
    S_ = _lib.Strides
    G = _lib.Geom
    fake = 4096  # never dereferenced: every call fails validation first
    st = lib.lcv_bsa_pool(None, 0, 1, 1, 64, 8, S_(512, 512, 8), G(4, 4, 4, 4, 4, 4), fake, None)
    assert st == _lib.ERR_INVALID_ARG
    st = lib.lcv_bsa_pool(fake, 0, 1, 1, 96, 8, S_(768, 768, 8), G(4, 4, 6, 4, 4, 4), fake, None)
    assert st == _lib.ERR_SHAPE and b"multiple of" in lib.lcv_bsa_last_error()
    st = lib.lcv_bsa_pool(fake, 0, 1, 1, 100, 8, S_(800, 800, 8), G(4, 4, 4, 4, 4, 4), fake, None)
    assert st == _lib.ERR_SHAPE and b"doesn't match" in lib.lcv_bsa_last_error()
    st = lib.lcv_bsa_pool(fake, 7, 1, 1, 64, 8, S_(512, 512, 8), G(4, 4, 4, 4, 4, 4), fake, None)
    assert st == _lib.ERR_DTYPE
    # Extents whose product overflows int64: rejected, not wrapped into a match.
    big = 1 << 40
    st = lib.lcv_bsa_pool(fake, 0, 1, 1, 64, 8, S_(512, 512, 8), G(big, big, 1 << 24, 4, 4, 4), fake, None)
    assert st == _lib.ERR_UNSUPPORTED
    st = lib.lcv_bsa_pool(fake, 0, 1, 1, 1 << 20, 8, S_(512, 512, 8),
                          G(1 << 30, 1 << 30, 4, 4, 4, 4), fake, None)
    assert st == _lib.ERR_SHAPE and b"doesn't match" in lib.lcv_bsa_last_error()
    st = lib.lcv_bsa_pool(fake, 0, big, big, 64, 8, S_(512, 512, 8), G(4, 4, 4, 4, 4, 4), fake, None)
    assert st == _lib.ERR_UNSUPPORTED
    args = dict(B=1, H=1, S=64, D=128)
    st = lib.lcv_bsa_attn_fwd(fake, fake, fake, 0, 1, 1, 64, 128, S_(8192, 8192, 128),
                              S_(8192, 8192, 128), S_(8192, 8192, 128), fake, None, 0, 0.1,
                              G(4, 4, 4, 4, 4, 4), fake, S_(8192, 8192, 128), None)
    assert st == _lib.ERR_INVALID_ARG  # top_k = 0
    st = lib.lcv_bsa_attn_fwd(fake, fake, fake, 0, 1, 1, 8, 128, S_(1024, 1024, 128),
                              S_(1024, 1024, 128), S_(1024, 1024, 128), fake, None, 1, 0.1,
                              G(2, 2, 2, 2, 2, 2), fake, S_(1024, 1024, 128), None)
    assert st == _lib.ERR_UNSUPPORTED and b"64-token" in lib.lcv_bsa_last_error()
    st = lib.lcv_bsa_attn_fwd(fake, fake, fake, 0, 1, 1, 64, 24, S_(1536, 1536, 24),
                              S_(1536, 1536, 24), S_(1536, 1536, 24), fake, None, 1, 0.1,
                              G(4, 4, 4, 4, 4, 4), fake, S_(1536, 1536, 24), None)
    assert st == _lib.ERR_UNSUPPORTED and b"head_dim" in lib.lcv_bsa_last_error()
    st = lib.lcv_bsa_attn_fwd(fake + 2, fake, fake, 0, 1, 1, 64, 128, S_(8192, 8192, 128),
                              S_(8192, 8192, 128), S_(8192, 8192, 128), fake, None, 1, 0.1,
                              G(4, 4, 4, 4, 4, 4), fake, S_(8192, 8192, 128), None)
    assert st == _lib.ERR_LAYOUT
    st = lib.lcv_bsa_attn_fwd(fake, fake, fake, 0, 1, 1, 64, 128, S_(8192, 8192, 64),
                              S_(8192, 8192, 128), S_(8192, 8192, 128), fake, None, 1, 0.1,
                              G(4, 4, 4, 4, 4, 4), fake, S_(8192, 8192, 128), None)
    assert st == _lib.ERR_LAYOUT  # row stride below D
    st = lib.lcv_bsa_topk(fake, 1, 1, 4, 8, 9, fake, None)
    assert st == _lib.ERR_INVALID_ARG  # top_k > nk
    st = lib.lcv_bsa_select(fake, fake, 1, 1, 4, 5000, 64, 4, fake, None)
    assert st == _lib.ERR_UNSUPPORTED  # nk > 4096
    st = lib.lcv_bsa_select(fake, fake, 1, 1, 4, 8, 6, 4, fake, None)
    assert st == _lib.ERR_UNSUPPORTED  # D % 4
    ws = lib.lcv_bsa_forward_workspace_bytes(1, 32, 900, 128)
    # pooled q and k means, block scores, launch order (each 256-byte aligned)
    assert ws == 2 * 32 * 900 * 128 * 4 + 32 * 900 * 900 * 4 + (32 * 900 * 4 + 255) // 256 * 256
    st = lib.lcv_bsa_schedule(fake, 1, 1, 5000, 4, fake, None)
    assert st == _lib.ERR_UNSUPPORTED  # nq > 4096
    st = lib.lcv_bsa_forward(fake, fake, fake, 0, 1, 1, 4096, 128, S_(1 << 19, 1 << 19, 128),
                             S_(1 << 19, 1 << 19, 128), S_(1 << 19, 1 << 19, 128), 4, 0.1,
                             G(1, 1, 4096, 1, 1, 64), fake, 16, fake, fake,
                             S_(1 << 19, 1 << 19, 128), None)
    assert st == _lib.ERR_INVALID_ARG and b"workspace" in lib.lcv_bsa_last_error()
    with pytest.raises(ValueError, match="multiple of"):
        _lib.check(lib.lcv_bsa_pool(fake, 0, 1, 1, 96, 8, S_(768, 768, 8), G(4, 4, 6, 4, 4, 4),
                                    fake, None), "pool")


@pytest.mark.skipif(not NO_GPU, reason="validation-only calls use fake pointers; CPU container only")
def test_noalloc_validation_returns_before_launch():
    """lcv_bsa_forward_noalloc refuses, before touching the device: a launch
    order beyond its 1 MiB array, an out with gaps between its elements, and
    an out overlapping q, k, v or idx (it stages the means and scores in out).
    A dense out in [B, S, H, D] order passes every check and reaches the
    first runtime call, which fails here without a GPU."""
    from lcv_bsa import _lib

    lib = _lib.load()
    S_, G = _lib.Strides, _lib.Geom
    assert _lib.NOALLOC_SCRATCH_BYTES == 1 << 20
    gib = 1 << 30  # fake, 16-byte aligned, never dereferenced
    q, k, v, out, idx = 1 * gib, 2 * gib, 3 * gib, 4 * gib, 5 * gib
    B, H, S, D, top_k = 1, 4, 4096, 128, 4
    dense = S_(H * S * D, S * D, D)

    def call(out=out, os=dense, q=q, idx=idx, B=B, H=H, S=S, qs=None):
        qs = qs or S_(H * S * D, S * D, D)
        return lib.lcv_bsa_forward_noalloc(q, k, v, _lib.F16, B, H, S, D, qs, qs, qs, top_k, 0.1,
                                           G(1, 1, S, 1, 1, 64), idx, out, os, None)

    # B*H*nb = 8 * 40 * 900 = 288,000 int32 > 1 MiB
    st = call(B=8, H=40, S=57600)
    assert st == _lib.ERR_UNSUPPORTED and b"fixed device scratch" in lib.lcv_bsa_last_error()
    assert call(os=S_(H * S * 2 * D, S * 2 * D, 2 * D)) == _lib.ERR_LAYOUT  # row gaps
    assert call(os=S_(2 * H * S * D, S * D, D), B=2) == _lib.ERR_LAYOUT  # batch gap
    assert b"dense" in lib.lcv_bsa_last_error()
    out_bytes = B * H * S * D * 2
    assert call(out=q) == _lib.ERR_INVALID_ARG and b"overlap" in lib.lcv_bsa_last_error()
    assert call(out=q + out_bytes - 16) == _lib.ERR_INVALID_ARG  # last row of q
    assert call(out=idx - out_bytes + 16) == _lib.ERR_INVALID_ARG  # first entries of idx
    # A batch stride of 2^62 elements: the inputs' spans pass every address
    # (computed without overflow), so they overlap out.
    assert call(B=2, os=S_(H * S * D, S * D, D), qs=S_(1 << 62, S * D, D)) == _lib.ERR_INVALID_ARG
    # Dense in [B, H, S, D] or [B, S, H, D] order (h stride D, s stride H*D),
    # also with q ending right where out starts: passes every check.
    for os, qq in ((dense, q), (S_(S * H * D, D, H * D), q), (dense, out - out_bytes)):
        assert call(os=os, q=qq) == _lib.ERR_LAUNCH
        assert b"hipStreamIsCapturing" in lib.lcv_bsa_last_error()


def test_prepare_qk_validation_and_table_length():
    """lcv_bsa_prepare_qk argument checks (no launch) and the table size."""
    from lcv_bsa import _lib, rope_table

    lib = _lib.load()
    S_, G, R = _lib.Strides, _lib.Geom, _lib.Grid
    n = lib.lcv_bsa_rope_table_len(128, R(16, 45, 80))
    assert n == 2 * (16 * 22 + 45 * 21 + 80 * 21)
    assert rope_table(128, (16, 45, 80)).numel() == n  # CPU tensor: same layout size
    assert lib.lcv_bsa_rope_table_len(64, R(2, 3, 4)) == 2 * (2 * 12 + 3 * 10 + 4 * 10)
    assert lib.lcv_bsa_rope_table_len(96, R(2, 3, 4)) == 0  # D unsupported
    assert lib.lcv_bsa_rope_table_len(128, R(64, 200, 300)) == 0  # table too large
    fake = 4096
    st_ = S_(4096 * 128, 4096 * 128, 128)
    g = G(1, 1, 4096, 1, 1, 64)

    def call(dtype=0, D=128, rope=R(4, 16, 64), tlen=None, geom=g, q=fake, eps=1e-6, strides=st_):
        tl = lib.lcv_bsa_rope_table_len(D, rope) if tlen is None else tlen
        return lib.lcv_bsa_prepare_qk(q, fake, dtype, 1, 1, 4096, D, strides, strides, None, None, eps,
                                      rope, fake, tl, geom, fake, fake, strides, strides, fake, fake, None)

    assert call(dtype=2) == _lib.ERR_UNSUPPORTED  # fp32
    assert call(dtype=9) == _lib.ERR_DTYPE
    assert call(D=96, strides=S_(4096 * 96, 4096 * 96, 96)) == _lib.ERR_UNSUPPORTED
    assert call(rope=R(4, 16, 32)) == _lib.ERR_SHAPE and b"RoPE grid" in lib.lcv_bsa_last_error()
    assert call(tlen=7) == _lib.ERR_INVALID_ARG and b"rope_table_len" in lib.lcv_bsa_last_error()
    assert call(geom=G(1, 2, 2048, 1, 2, 16)) == _lib.ERR_UNSUPPORTED  # 32-token blocks
    assert call(q=fake + 2) == _lib.ERR_LAYOUT
    assert call(eps=-1.0) == _lib.ERR_INVALID_ARG
    assert call(q=None) == _lib.ERR_INVALID_ARG


def test_python_api_rejects_cpu_tensors_loudly():
    """No silent CPU path: host tensors raise (not a ValueError, so the
    dispatcher cannot turn it into a dense fallback)."""
    from lcv_bsa import bsa_attention
    from lcv_bsa.block_sparse_attention import BSADeviceError

    q = torch.zeros((1, 1, 64, 16))
    with pytest.raises(BSADeviceError):
        bsa_attention(q, q, q, shape=(4, 4, 4))
    assert not issubclass(BSADeviceError, ValueError)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    from lcv_bsa import _lib

    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "missing.so")
    with pytest.raises(ImportError, match="no fallback"):
        _lib.load()


# ---------------------------------------------------------------------------
# Dispatcher and model wiring (test_bsa_dit_wiring_smoke.py)
# ---------------------------------------------------------------------------

class _Block:
    def __init__(self):
        from lcv_bsa import BSAAttention

        self.attn = BSAAttention(64, 4)


class _Model:
    def __init__(self, config):
        from lcv_bsa import BSAModelMixin, apply_bsa_params

        self.blocks = [_Block() for _ in range(config["depth"])]
        apply_bsa_params(self, config)

    def enable_bsa(self, backend="tier_a"):  # the reference's default (longcat_video_dit.py:219)
        from lcv_bsa import enable_bsa

        enable_bsa(self, backend)

    def disable_bsa(self):
        from lcv_bsa import disable_bsa

        disable_bsa(self)


def _config(enable=False):
    return {"depth": 2, "bsa_params": {"sparsity": 0.9375, "chunk_3d_shape_q": [4, 4, 4],
                                       "chunk_3d_shape_k": [4, 4, 4]}, "enable_bsa": enable}


def test_default_bsa_off():
    assert all(b.attn.enable_bsa is False for b in _Model(_config(False)).blocks)


def test_config_enable_bsa_flips_attention():
    m = _Model(_config(True))
    for b in m.blocks:
        assert b.attn.enable_bsa is True
        assert b.attn.bsa_sparsity == 0.9375 and b.attn.bsa_chunk_thw == (4, 4, 4)
        assert b.attn.bsa_backend == "tier_a"  # the reference's default name, served by HIP


def test_enable_disable_roundtrip():
    m = _Model(_config(False))
    m.enable_bsa()
    assert all(b.attn.enable_bsa for b in m.blocks)
    m.disable_bsa()
    assert not any(b.attn.enable_bsa for b in m.blocks)


def test_bsa_params_preserved_through_enable():
    cfg = _config(False)
    cfg["bsa_params"]["sparsity"] = 0.5
    cfg["bsa_params"]["chunk_3d_shape_q"] = [2, 2, 2]
    m = _Model(cfg)
    m.enable_bsa()
    assert all(b.attn.bsa_sparsity == 0.5 and b.attn.bsa_chunk_thw == (2, 2, 2) for b in m.blocks)


def test_backend_validation():
    """The reference's names (longcat_video_dit.py:249-252) are accepted and
    resolve to the HIP path; anything else is an AssertionError, as there."""
    from lcv_bsa.attention import resolve_backend, validate_backend

    for name in ("hip", "tier_a", "metal", "metal_v2", "metal_v3", "metal_v4"):
        assert validate_backend(name) == name
        assert resolve_backend(name) == "hip"
    for bad in ("cuda", "Tier_A", "metal_v5", ""):
        with pytest.raises(AssertionError, match="unknown BSA backend"):
            validate_backend(bad)
        with pytest.raises(AssertionError, match="unknown BSA backend"):
            resolve_backend(bad)
    m = _Model(_config(False))
    m.enable_bsa()  # the reference's default name
    assert all(b.attn.enable_bsa and b.attn.bsa_backend == "tier_a" for b in m.blocks)
    m.enable_bsa("metal_v4")
    assert all(b.attn.bsa_backend == "metal_v4" for b in m.blocks)
    with pytest.raises(AssertionError):
        m.enable_bsa("cuda")


def test_env_var_default_and_override(monkeypatch):
    """scripts/run_refine.py:91-92: unset -> "tier_a"; set -> that name."""
    from lcv_bsa.attention import backend_from_env
    from lcv_bsa.dit import enable_bsa_from_env

    monkeypatch.delenv("LONGCAT_BSA_BACKEND", raising=False)
    assert backend_from_env() == "tier_a"
    m = _Model(_config(False))
    assert enable_bsa_from_env(m) == "tier_a"
    assert all(b.attn.enable_bsa and b.attn.bsa_backend == "tier_a" for b in m.blocks)
    for name in ("hip", "metal"):
        monkeypatch.setenv("LONGCAT_BSA_BACKEND", name)
        assert backend_from_env() == name
    monkeypatch.setenv("LONGCAT_BSA_BACKEND", "mlx")
    with pytest.raises(AssertionError):
        enable_bsa_from_env(_Model(_config(False)))


def test_reference_backend_names_dispatch_on_cpu():
    """With a reference backend name the dispatcher takes the BSA branch; on
    CPU tensors the HIP path raises (there is no CPU fallback), while the
    dense path (shape None) still runs."""
    from lcv_bsa import BSAAttention
    from lcv_bsa.block_sparse_attention import BSADeviceError

    a = BSAAttention(2 * 64, 2)
    a.enable_bsa, a.bsa_backend = True, "tier_a"
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 2, 64, 64, generator=g) for _ in range(3))
    with pytest.raises(BSADeviceError):
        a._process_attn(q, k, v, shape=(1, 1, 64))
    out = a._process_attn(q, k, v, shape=None)
    assert a.last_path == "dense" and out.shape == q.shape
    a.bsa_backend = "cuda"
    with pytest.raises(AssertionError):
        a._process_attn(q, k, v, shape=(1, 1, 64))


def test_process_attn_dense_path_on_cpu():
    """BSA off, or shape None: dense SDPA with scale head_dim**-0.5 (attention.py:179)."""
    from lcv_bsa import BSAAttention

    a = BSAAttention(4 * 16, 4)
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 4, 64, 16, generator=g) for _ in range(3))
    out = a._process_attn(q, k, v, shape=(4, 4, 4))
    assert a.last_path == "dense"
    ref = O.sdpa(q.numpy(), k.numpy(), v.numpy(), 0.25)
    assert np.abs(out.numpy() - ref).max() < 1e-5
    a.enable_bsa = True
    out = a._process_attn(q, k, v, shape=None)
    assert a.last_path == "dense"


# ---------------------------------------------------------------------------
# Count rules and the workload generator
# ---------------------------------------------------------------------------

def test_count_rules():
    from lcv_bsa import num_selected_blocks
    from lcv_bsa.workloads import top_k_ceil, top_k_floor

    assert num_selected_blocks(900, 0.9375) == 56 == top_k_floor(900, 0.9375)
    assert top_k_ceil(900, 0.9375) == 57 and top_k_ceil(450, 0.9375) == 29
    assert [top_k_ceil(900, s) for s in (0.875, 0.9375, 0.96875)] == [113, 57, 29]
    assert [top_k_floor(900, s) for s in (0.875, 0.9375, 0.96875)] == [112, 56, 28]
    assert top_k_ceil(8, 0.75) == 2 and top_k_floor(4, 0.99) == 1


def test_executed_flops_headline():
    from lcv_bsa.workloads import executed_flops

    f = executed_flops(1, 32, 900, 57, 128)
    assert f == 4 * 32 * 900 * 57 * 64 * 64 * 128
    assert abs(f / 1e12 - 3.4427) < 1e-3
    assert abs(executed_flops(1, 32, 450, 29, 128) / 1e12 - 0.8758) < 1e-3


def test_block_tokens_matches_oracle():
    from lcv_bsa.workloads import block_tokens

    for shape, chunk in [((8, 12, 16), (4, 4, 4)), ((1, 1, 512), (1, 1, 64)), ((4, 6, 8), (2, 3, 4))]:
        assert np.array_equal(block_tokens(shape, chunk).numpy(), O.block_tokens(shape, chunk))


def test_rope_matches_oracle():
    from lcv_bsa.rope_3d import rope_3d, rope_freqs_3d, rope_dims

    assert rope_dims(128) == (44, 42, 42)
    grid = (3, 5, 7)
    f = rope_freqs_3d(grid, 128).numpy()
    fo = O.rope_freqs_3d(grid, 128)
    assert np.allclose(f, fo, rtol=1e-6, atol=1e-6)
    g = torch.Generator().manual_seed(0)
    q = torch.randn(1, 2, 105, 128, generator=g)
    qr, _ = rope_3d(q, q, grid)
    assert np.allclose(qr.numpy(), O.apply_rope(q.numpy(), fo), atol=2e-5)


def test_inputs_margins_and_determinism():
    from lcv_bsa.workloads import make_inputs

    shape, chunk, ks = (1, 1, 4096), (1, 1, 64), (3, 4)
    q, k, v, info = make_inputs(1, 2, 64, shape, chunk, torch.float16, "cpu", seed=5,
                                grid=(4, 16, 64), margin_ks=ks)
    q2, k2, v2, _ = make_inputs(1, 2, 64, shape, chunk, torch.float16, "cpu", seed=5,
                                grid=(4, 16, 64), margin_ks=ks)
    assert torch.equal(q, q2) and torch.equal(k, k2) and torch.equal(v, v2)
    assert q.dtype == torch.float16
    sc = O.block_routing_scores(O.mean_pool_blocks_3d(q.float().numpy(), shape, chunk),
                                O.mean_pool_blocks_3d(k.float().numpy(), shape, chunk))
    top = -np.sort(-sc, axis=-1)
    for kk in ks:
        assert (top[..., kk - 1] - top[..., kk]).min() > 1e-4
    print("repairs", info["repairs"], "rounds", info["rounds"])


def test_inputs_voxel_geometry_offsets():
    """The low-rank offset is added per voxel block (block_tokens mapping)."""
    from lcv_bsa.workloads import make_inputs

    shape, chunk = (8, 8, 8), (4, 4, 4)
    q, k, v, info = make_inputs(1, 1, 32, shape, chunk, torch.float32, "cpu", seed=1,
                                offset_std=50.0)
    qb = O.mean_pool_blocks_3d(q.numpy(), shape, chunk)
    # the offset dominates each voxel's mean; rows of one voxel share it
    bt = O.block_tokens(shape, chunk)
    U = info["U"].numpy()
    for n in range(bt.shape[0]):
        proj = q.numpy()[0, 0, bt[n]] @ U.T  # [64, 4]
        assert np.abs(proj.mean(0) - qb[0, 0, n] @ U.T).max() < 1e-3
        assert proj.std(0).max() < 3.0  # N(0,1) noise around a shared offset


# ---------------------------------------------------------------------------
# Golden fixtures: the oracle and the generator still reproduce them
# ---------------------------------------------------------------------------

def test_golden_c0_reproduced():
    from lcv_bsa.workloads import make_workload

    fx = np.load(REPO / "tests" / "golden" / "c0.npz")
    w = make_workload("c0", "cpu", seed=int(fx["seed"]))
    assert float(w.q.double().sum()) == pytest.approx(float(fx["q_sum"]), abs=1e-6)
    q, k, v = (t.numpy() for t in (w.q, w.k, w.v))
    out, idx = O.bsa_attention(q, k, v, w.shape, 0.9375, w.chunk_thw, top_k=int(fx["top_k"]),
                               return_indices=True)
    assert np.array_equal(idx, fx["indices"])
    assert np.abs(out[:, :, fx["rows"]] - fx["out_rows"]).max() < 1e-12


def test_golden_voxel_reproduced():
    fx = np.load(REPO / "tests" / "golden" / "voxel.npz")
    shape, chunk = tuple(fx["shape"]), tuple(fx["chunk"])
    q, k, v = (fx[n].astype(np.float32) for n in ("q", "k", "v"))
    out, idx = O.bsa_attention_masked(q, k, v, shape, float(fx["sparsity"]), chunk,
                                      return_indices=True)
    assert np.array_equal(idx, fx["indices"])
    assert np.abs(out - fx["out"]).max() < 1e-6


# ---------------------------------------------------------------------------
# Shape policy and the DiT block's host side
# ---------------------------------------------------------------------------

def test_shape_policy_decisions():
    from lcv_bsa.shape_policy import bsa_geometry

    g720 = (16, 45, 80)
    # The reference keeps (shape, chunk): BSA then raises ValueError -> dense.
    assert bsa_geometry(g720, (4, 4, 4), "reference") == (g720, (4, 4, 4))
    with pytest.raises(ValueError):
        O.mean_pool_blocks_3d(np.zeros((1, 1, 57600, 8)), g720, (4, 4, 4))
    # auto: the voxel where it tiles, else 64-token runs, else dense.
    assert bsa_geometry((16, 48, 80), (4, 4, 4), "auto") == ((16, 48, 80), (4, 4, 4))
    assert bsa_geometry(g720, (4, 4, 4), "auto") == ((1, 1, 57600), (1, 1, 64))
    assert bsa_geometry((1, 3, 7), (4, 4, 4), "auto") is None
    assert bsa_geometry((16, 48, 80), (4, 4, 4), "contiguous") == ((1, 1, 61440), (1, 1, 64))
    with pytest.raises(ValueError):
        bsa_geometry(g720, (4, 4, 4), "pad")


def test_dit_block_parameters_match_checkpoint_layout():
    """Module and parameter names / shapes of the torch block are the
    reference's (PyTorch checkpoint keys, longcat_video_dit.py:36-66), with
    the SwiGLU width 11008 at dim 4096."""
    from oracle.dit_block_oracle import block_param_shapes

    from lcv_bsa.dit_block import LongCatSingleStreamBlock

    with torch.device("meta"):
        blk = LongCatSingleStreamBlock(4096, 32, 4, 512)
    sd = {k: tuple(v.shape) for k, v in blk.state_dict().items()}
    assert sd == block_param_shapes(4096, 32, 4, 512)
    assert blk.ffn.hidden_dim == 11008
    assert blk.attn.bsa_shape_policy == "reference" and not blk.attn.enable_bsa


def test_dit_block_reference_modulation_asserts_fp32():
    from lcv_bsa.dit_block import LayerNorm_FP32, modulate_fp32

    norm = LayerNorm_FP32(8, 1e-6, elementwise_affine=False)
    x = torch.randn(1, 2, 3, 8)
    zero = torch.zeros(1, 2, 1, 8)
    y = modulate_fp32(norm, x, zero, zero)
    assert torch.allclose(y, torch.nn.functional.layer_norm(x, (8,), eps=1e-6), atol=1e-6)
    with pytest.raises(AssertionError):
        modulate_fp32(norm, x, zero.to(torch.bfloat16), zero)


def test_bench_refuses_more_than_one_gpu():
    """bench.py runs the single-GPU path only: --gpus 2 exits with status 2
    and says why, before touching a device."""
    import json
    import subprocess
    import sys

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], cwd=root,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


@pytest.mark.parametrize("lang,std", [("c", "c99"), ("c++", "c++17")])
def test_header_compiles_for_c_and_cpp_callers(tmp_path, lang, std):
    """include/lcv_bsa.h is a plain C-ABI header: it compiles warning-free as
    C99 and as C++17 (the bindings of a cgo / JNI / N-API / ctypes caller)."""
    import shutil
    import subprocess

    cc = shutil.which("gcc" if lang == "c" else "g++")
    if cc is None:
        pytest.skip("no host compiler")
    src = tmp_path / "use_header.c"
    src.write_text('#include "lcv_bsa.h"\nint main(void) { return lcv_bsa_version() ? 0 : 1; }\n')
    r = subprocess.run([cc, "-x", lang, f"-std={std}", "-Wall", "-Wextra", "-pedantic", "-Werror",
                        f"-I{REPO / 'include'}", "-fsyntax-only", str(src)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr


def test_gathered_reference_matches_oracle():
    """The fp32 torch reference that the full-size GPU tests compare every
    q-block with equals the fp64 oracle on a small routed case (unsorted
    lists included), and a planted key transpose in it is caught."""
    from conftest import gathered_attention_fp32

    g = torch.Generator().manual_seed(3)
    B, H, S, D, k = 2, 3, 1024, 32, 5
    q, kk, v = (torch.randn(B, H, S, D, generator=g) for _ in range(3))
    nb = S // 64
    idx = torch.stack([torch.randperm(nb, generator=g)[:k] for _ in range(B * H * nb)]).reshape(B, H, nb, k)
    idx = idx.to(torch.int32)
    got = gathered_attention_fp32(q, kk, v, idx, 0.3, step=5).numpy()
    ref = O.sparse_attention_from_indices(q.numpy(), kk.numpy(), v.numpy(), idx.numpy(), (1, 1, S),
                                          (1, 1, 64), 0.3)
    assert np.abs(got - ref).max() < 2e-5
    wrong = gathered_attention_fp32(q, kk.transpose(2, 3).reshape(B, H, S, D), v, idx, 0.3).numpy()
    assert np.abs(wrong - ref).max() > 1e-2
