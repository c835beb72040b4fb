"""Writes the golden fixtures under tests/golden/ from the oracle.

c0.npz    -- config 0 (B1 H2 S4096 D64 fp32, contiguous 64-token blocks,
             top-k 4): the routing [1,2,64,4] and every 16th output row in
             fp64, plus the input checksum (inputs are regenerated from the
             seed by lcv_bsa.workloads on the CPU).
voxel.npz -- a small complete case with (4,4,4) voxels: fp16 inputs
             [1,2,512,32], routing and fp64 output.

The reference (MLX) cannot run here, so the vectors come from the oracle
(oracle/bsa_oracle.py), itself pinned by tests/test_oracle.py.  Usage:
    python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
for p in (str(REPO), str(REPO / "longcat-video-mlx_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import torch  # noqa: E402

from lcv_bsa.workloads import make_inputs, make_workload  # noqa: E402
from oracle import bsa_oracle as O  # noqa: E402


def make_c0(seed: int = 0) -> None:
    w = make_workload("c0", "cpu", seed=seed)
    q, k, v = (t.numpy() for t in (w.q, w.k, w.v))
    out, idx = O.bsa_attention(q, k, v, w.shape, 0.9375, w.chunk_thw, top_k=w.top_k,
                               return_indices=True)
    masked = O.bsa_attention_masked(q, k, v, w.shape, 0.9375, w.chunk_thw, top_k=w.top_k)
    assert np.abs(out - masked).max() < 1e-12
    rows = np.arange(0, q.shape[2], 16)
    np.savez_compressed(HERE / "c0.npz", seed=seed, top_k=w.top_k, q_sum=float(w.q.double().sum()),
                        indices=idx, rows=rows, out_rows=out[:, :, rows],
                        torch_version=torch.__version__)
    print(f"c0: repairs={w.repairs} indices {idx.shape} rows {rows.size}")


def make_voxel(seed: int = 3) -> None:
    shape, chunk = (8, 8, 8), (4, 4, 4)
    q, k, v, info = make_inputs(1, 2, 32, shape, chunk, torch.float16, "cpu", seed=seed,
                                grid=shape, margin_ks=(2, 3))
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    out, idx = O.bsa_attention(qn, kn, vn, shape, 0.75, chunk, return_indices=True)
    np.savez_compressed(HERE / "voxel.npz", q=q.numpy(), k=k.numpy(), v=v.numpy(),
                        shape=np.array(shape), chunk=np.array(chunk), sparsity=0.75,
                        indices=idx, out=out.astype(np.float32))
    print(f"voxel: repairs={info['repairs']} indices {idx.shape}")


if __name__ == "__main__":
    make_c0()
    make_voxel()
