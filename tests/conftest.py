"""Shared test setup: import paths, the ``gpu`` marker, small helpers."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
PKG_ROOT = REPO / "longcat-video-mlx_amd"
for p in (str(REPO), str(PKG_ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (gfx950) device; runs the HIP kernels")


@pytest.fixture(scope="session")
def device():
    """cuda:0 with the native library loaded.  GPU tests fail (not skip) on a
    machine without a device, so they can never pass silently."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no ROCm device is visible")
    from lcv_bsa import _lib

    _lib.load()  # raises if liblcv_bsa.so is missing
    return torch.device("cuda", 0)


def assert_close_report(actual, expected, max_abs: float, mean_abs: float, what: str = ""):
    """max-abs / mean-abs parity check with a readable report."""
    import numpy as np

    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    assert a.shape == e.shape, f"{what}: shape {a.shape} != {e.shape}"
    assert np.isfinite(a).all(), f"{what}: non-finite values in result"
    d = np.abs(a - e)
    mx, mn = float(d.max()), float(d.mean())
    assert mx <= max_abs and mn <= mean_abs, (
        f"{what}: max_abs={mx:.3e} (tol {max_abs:.1e}) mean_abs={mn:.3e} (tol {mean_abs:.1e})")
    return mx, mn


def gathered_attention_fp32(q, k, v, idx, scale, step=128):
    """fp32 attention of every q-block over its listed 64-token K/V blocks of
    contiguous-run geometry (shape (1, 1, S), chunk (1, 1, 64)), in torch on
    q's device: gather, fp32 scores, softmax, fp32 P V.  Shares no code with
    the HIP kernels; pinned against the NumPy oracle by
    test_cpu_host.py::test_gathered_reference_matches_oracle."""
    import torch

    B, H, S, D = q.shape
    nb, top_k = S // 64, idx.shape[-1]
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    for b in range(B):
        for h in range(H):
            qh = q[b, h].float().reshape(nb, 64, D)
            kh = k[b, h].float().reshape(-1, 64, D)
            vh = v[b, h].float().reshape(-1, 64, D)
            ih = idx[b, h].long()
            for n0 in range(0, nb, step):
                n = min(step, nb - n0)
                ii = ih[n0:n0 + n]
                kt = kh[ii].reshape(n, top_k * 64, D).transpose(1, 2).contiguous()
                vg = vh[ii].reshape(n, top_k * 64, D).contiguous()
                p = torch.softmax(torch.bmm(qh[n0:n0 + n].contiguous(), kt) * scale, dim=-1)
                out[b, h, n0 * 64:(n0 + n) * 64] = torch.bmm(p, vg).reshape(n * 64, D)
    return out


def wide_range_inputs(D: int, q_scale: float, dtype, seeds=(31, 32, 33), wide_rows=None):
    """Inputs of the wide-score-range attention tests, built on the CPU:
    q ~ N(0,1) scaled by q_scale (only on rows wide_rows[0] <= r % 64 <
    wide_rows[1] when given), K block j scaled by 1 + j/4 (scores grow along
    the list), v ~ N(0,1), rounded to ``dtype``; two heads over S = 2048
    (32 blocks of 64), every q-block routed to the even blocks, ascending in
    head 0 and descending in head 1.  Returns (q, k, v, idx [1,2,32,16])."""
    import numpy as np
    import torch

    def rand(shape, seed):
        g = torch.Generator(device="cpu").manual_seed(seed)
        return torch.randn(*shape, generator=g)

    nb = 32
    q = rand((1, 2, 2048, D), seeds[0])
    if wide_rows is None:
        q = q * q_scale
    else:
        rows = torch.arange(2048) % 64
        q = q * torch.where((rows >= wide_rows[0]) & (rows < wide_rows[1]), q_scale, 1.0)[None, None, :, None]
    k = rand((1, 2, 2048, D), seeds[1])
    k = k * (1.0 + torch.arange(2048).div(64, rounding_mode="floor").float() / 4.0)[None, None, :, None]
    v = rand((1, 2, 2048, D), seeds[2])
    idx = np.broadcast_to(np.arange(0, nb, 2, dtype=np.int32), (1, 2, nb, nb // 2)).copy()
    idx[0, 1] = idx[0, 1, :, ::-1]  # descending lists too
    return q.to(dtype), k.to(dtype), v.to(dtype), idx
