"""Benchmark: Block Sparse Attention forward at the 720p refinement shape.

Default workload (one MI355X): B=1, 32 heads, S=57600 (16 x 45 x 80 latent
grid, contiguous 64-token blocks -> 900 blocks), D=128, fp16, top-k = 57 KV
blocks per q-block (ceil(0.0625 * 900); the reference's floor rule gives 56).
Inputs are synthetic (seeded N(0,1) + per-block low-rank offsets, 3D RoPE,
margin-repaired routing) and resident in HBM before timing starts.

One step = one full BSA forward through the C ABI (pool q/k -> fused scores +
top-k -> sparse attention), timed with HIP events on the launch stream.  A
second timed pass launches the three stages separately to attribute time per
kernel; the attention kernel's average duration gives the roofline line.

Prints ONE JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import re
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (str(REPO), str(REPO / "longcat-video-mlx_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "BSA fwd ms + executed-block TFLOP/s (% fp16 MFMA peak), S=57600 32h D128"
PEAK_TFLOPS = {"f16": 2500.0, "bf16": 2500.0}  # MI355X dense MFMA peak
DTYPE_NAME = {"float16": "f16", "bfloat16": "bf16", "float32": "f32"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def _traffic_from_profiles(workload: str):
    """HBM bytes per attention launch from the committed rocprofv3 PMC summary."""
    p = REPO / "profiles" / f"attn_fwd_{workload}_traffic.txt"
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


def _cpu_model() -> str:
    """The host CPU as /proc/cpuinfo names it, with its x86 family / model
    numbers (virtual machines often report only a generic model name) and
    the hypervisor flag."""
    fields = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" not in line:
                if fields:
                    break  # first processor's block only
                continue
            key, val = (s.strip() for s in line.split(":", 1))
            fields.setdefault(key, val)
    except OSError:
        pass
    name = fields.get("model name") or platform.processor() or platform.machine()
    extra = []
    if "cpu family" in fields and "model" in fields:
        fam, model = fields["cpu family"], fields["model"]
        extra.append(f"x86 family {fam} model {model}")
        if fields.get("vendor_id") == "AuthenticAMD" and fam == "26":
            extra.append("Zen 5")
    if "hypervisor" in fields.get("flags", "").split():
        extra.append("virtual machine")
    return f"{name} ({', '.join(extra)})" if extra else name


def cpu_baseline(w, budget_s: float):
    """The oracle (fp32 NumPy restatement of Tier A) on a bounded sample of the
    same workload: pooling + routing for the sampled heads, then the gathered
    attention for their q-blocks, until ``budget_s`` of CPU time is spent."""
    import numpy as np

    from oracle import bsa_oracle as O

    host_cpus = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):  # pragma: no cover - non-Linux
        avail = host_cpus
    # Every core this process may run on, within the per-GPU CPU share the
    # job's launcher sets through OMP_NUM_THREADS (a shared host's other
    # GPUs' jobs keep theirs).
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads = min(avail, share) if share > 0 else avail
    limiter = None
    try:
        from threadpoolctl import threadpool_info, threadpool_limits
        limiter = threadpool_limits(limits=threads, user_api="blas")
        threads = max(int(i.get("num_threads", 1)) for i in threadpool_info() if i.get("user_api") == "blas")
    except Exception:  # pragma: no cover - threadpoolctl is optional
        pass
    B, H, S, D = w.q.shape
    nb = S // 64
    k = w.top_k
    done_blocks, heads, t_total = 0, 0, 0.0
    for b in range(B):
        for h in range(H):
            qh = w.q[b:b + 1, h:h + 1].float().cpu().numpy()
            kh = w.k[b:b + 1, h:h + 1].float().cpu().numpy()
            vh = w.v[b:b + 1, h:h + 1].float().cpu().numpy()
            t0 = time.perf_counter()
            qbar = O.mean_pool_blocks_3d(qh, w.shape, w.chunk_thw, acc=np.float32)
            kbar = O.mean_pool_blocks_3d(kh, w.shape, w.chunk_thw, acc=np.float32)
            idx, _ = O.topk_block_indices(O.block_routing_scores(qbar, kbar, acc=np.float32), top_k=k)
            t_total += time.perf_counter() - t0
            heads += 1
            step = 64
            for n0 in range(0, nb, step):
                t0 = time.perf_counter()
                O.sparse_attention_from_indices(qh, kh, vh, idx, w.shape, w.chunk_thw, w.sm_scale,
                                                acc=np.float32, q_blocks=np.arange(n0, min(nb, n0 + step)))
                t_total += time.perf_counter() - t0
                done_blocks += min(nb, n0 + step) - n0
                if t_total >= budget_s:
                    break
            if t_total >= budget_s:
                break
        if t_total >= budget_s:
            break
    if limiter is not None:
        limiter.restore_original_limits()
    flops = O.executed_flops(1, 1, done_blocks, k, D)
    cpu = _cpu_model()
    return {
        "value": flops / t_total / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "host_cpus": host_cpus,
        "available_cpus": avail,
        "cpu_model": cpu,
        "sample": (f"oracle fp32 (NumPy/OpenBLAS) on {threads} threads = every CPU available to the "
                   f"process ({avail} of the host's {host_cpus}, {cpu}) within the per-GPU share "
                   f"OMP_NUM_THREADS={share or 'unset'}: pool+route of {heads} head(s) and sparse "
                   f"attention of {done_blocks} q-blocks x {k} KV blocks in {t_total:.1f} s; "
                   f"full-workload estimate {t_total * (B * H * nb) / max(done_blocks, 1):.0f} s"),
    }


def bench_prepare(lib, w, dev, stream, steps: int, warmup: int, seed: int):
    """The fused pre-BSA pass (RMSNorm + 3D RoPE of q and k, block means) at the
    workload's shape, fed the way the DiT feeds it: q / k are [B, H, S, D]
    views of a fused QKV output [B, S, 3, H, D] (attention.py:191-201).

    HBM-bound: per (q or k, batch, head, 64-token block) it reads and writes
    64 x D elements and writes D fp32 means.  The reference's unfused chain
    (fp32 RMSNorm -> rounded -> weight -> fp32 RoPE -> rounded, then the
    pooling) is timed beside it in torch on the same GPU."""
    import torch

    from lcv_bsa import _lib
    from lcv_bsa.block_sparse_attention import _geom, _strides
    from lcv_bsa.prepare import RMS_EPS, rope_table
    from lcv_bsa.rope_3d import rope_freqs_3d, rotate_half

    B, H, S, D = w.q.shape
    nb = w.num_blocks
    dt = w.q.dtype
    code = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}[dt]
    gen = torch.Generator(device=dev).manual_seed(seed + 1)
    qkv = torch.randn((B, S, 3, H, D), generator=gen, device=dev, dtype=torch.float32).to(dt)
    q, k = qkv[:, :, 0].transpose(1, 2), qkv[:, :, 1].transpose(1, 2)
    wq = (1.0 + 0.1 * torch.randn(D, generator=gen, device=dev)).to(dt)
    wk = (1.0 + 0.1 * torch.randn(D, generator=gen, device=dev)).to(dt)
    grid = _lib.Grid(*(int(x) for x in w.grid))
    n_tab = lib.lcv_bsa_rope_table_len(D, grid)
    table = rope_table(D, w.grid, dev)
    q_out, k_out = torch.empty((B, H, S, D), dtype=dt, device=dev), torch.empty((B, H, S, D), dtype=dt, device=dev)
    qb = torch.empty((B, H, nb, D), dtype=torch.float32, device=dev)
    kb = torch.empty_like(qb)
    geom = _geom(w.shape, w.chunk_thw)
    sh = stream.cuda_stream

    def fused():
        _lib.check(lib.lcv_bsa_prepare_qk(
            q.data_ptr(), k.data_ptr(), code, B, H, S, D, _strides(q), _strides(k), wq.data_ptr(),
            wk.data_ptr(), RMS_EPS, grid, table.data_ptr(), n_tab, geom, q_out.data_ptr(),
            k_out.data_ptr(), _strides(q_out), _strides(k_out), qb.data_ptr(), kb.data_ptr(), sh),
            "prepare_qk")

    f = rope_freqs_3d(tuple(w.grid), D, dev)
    cos, sin = torch.cos(f), torch.sin(f)

    def unfused():
        outs = []
        for x, wt in ((q, wq), (k, wk)):
            xf = x.float()
            y = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + RMS_EPS)).to(dt) * wt
            yf = y.float()
            r = (yf * cos + rotate_half(yf) * sin).to(dt)
            outs.append(r.reshape(B, H, nb, 64, D).float().mean(3))
        return outs

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    # The box's own device-to-device copy of the bytes prepare_qk streams
    # (q and k read once, written once): the practical rate of a read+write
    # HBM pass on this GPU, timed in the same run.
    esz = q.element_size()
    half = 2 * B * H * S * D * esz
    src = torch.empty((half,), dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)

    def copy():
        dst.copy_(src)

    for _ in range(warmup):
        fused()
        copy()
    ms = timed(fused, steps)
    ms_copy = timed(copy, steps)
    unfused()
    ms_torch = timed(unfused, max(2, steps // 4))
    nbytes = 2 * B * H * nb * (2 * 64 * D * esz + D * 4)
    gbs = nbytes / (ms * 1e-3) / 1e9
    copy_gbs = 2 * half / (ms_copy * 1e-3) / 1e9
    del qkv, q_out, k_out, src, dst
    torch.cuda.empty_cache()
    return {
        "kernel": "prep_kernel",
        "inputs": f"q, k as [B,H,S,D] views of a [B,S,3,H,D] {DTYPE_NAME[str(dt).split('.')[1]]} QKV buffer, "
                  f"RoPE grid {tuple(w.grid)}",
        "ms": round(ms, 4),
        "algorithmic_bytes": nbytes,
        "achieved": round(gbs, 1),
        "peak": 8000.0,
        "unit": "GB/s",
        "frac": round(gbs / 8000.0, 4),
        "copy": {"what": f"device-to-device copy of {half} B (torch copy_, hipMemcpyAsync), "
                         f"{2 * half} B of reads + writes", "ms": round(ms_copy, 4),
                 "achieved": round(copy_gbs, 1), "unit": "GB/s"},
        "frac_of_copy": round(gbs / copy_gbs, 4),
        "unfused_torch_ms": round(ms_torch, 4),
    }


def bench_dit_block(dev, stream, steps: int, warmup: int, seed: int, top_k: int, dtype=None):
    """One LongCat DiT block at 720p (longcat_video_dit.py:36-138): hidden
    4096, 32 heads of 128, SwiGLU inner 11008, AdaLN from a 512-wide timestep
    embedding per frame, 512 text tokens, latent grid 16 x 45 x 80, fp16
    activations (or ``dtype``), random weights.  The self-attention runs the fused pre-BSA pass and BSA
    (64-token blocks, top-k ``top_k``); the linear layers are torch GEMMs.

    A first timed region runs whole blocks; a second attributes time to the
    sub-modules with events recorded by forward hooks.  The BSA share is the
    self-attention minus its two GEMMs: prepare_qk + routing + attention."""
    import torch

    from lcv_bsa.dit_block import LongCatSingleStreamBlock

    dt = torch.float16 if dtype is None else dtype
    grid, C, H, L, t_dim = (16, 45, 80), 4096, 32, 512, 512
    N = grid[0] * grid[1] * grid[2]
    torch.manual_seed(seed + 2)
    blk = LongCatSingleStreamBlock(C, H, 4, t_dim, dtype=dt, device=dev)
    with torch.no_grad():
        for name, p in blk.named_parameters():
            if name.endswith("norm.weight") or name == "pre_crs_attn_norm.weight":
                p.fill_(1.0)
            else:
                p.normal_(0.0, 0.02)
    blk.attn.enable_bsa, blk.attn.bsa_shape_policy, blk.attn.bsa_top_k = True, "auto", top_k
    gen = torch.Generator(device=dev).manual_seed(seed + 3)
    x = torch.randn((1, N, C), generator=gen, device=dev).to(dt)
    y = torch.randn((1, L, C), generator=gen, device=dev).to(dt)
    t = torch.randn((1, grid[0], t_dim), generator=gen, device=dev)

    def step():
        with torch.no_grad():
            return blk(x, y, t, [L], grid)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    assert blk.attn.last_path == "bsa"

    marks: dict = {}
    mods = {"self_attn": blk.attn, "qkv_gemm": blk.attn.qkv, "proj_gemm": blk.attn.proj,
            "cross_attn": blk.cross_attn, "pre_cross_norm": blk.pre_crs_attn_norm, "ffn": blk.ffn}
    handles = []
    # The two library calls between the QKV and proj GEMMs, timed the same
    # way: prepare_qk (RMSNorm + RoPE + block means) and bsa_attention
    # (routing from the means, launch order, attention kernel).
    import lcv_bsa.dit_block as dbm
    wrapped = {"prepare_qk": dbm.prepare_qk, "bsa_attention": dbm.bsa_attention}

    seen: dict = {}

    def timed_call(name, fn):
        def run(*a, **kw):
            e0_, e1_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0_.record(stream)
            r = fn(*a, **kw)
            e1_.record(stream)
            marks.setdefault(name, []).append([e0_, e1_])
            seen[name] = (a, kw, r)
            return r
        return run
    for name, fn in wrapped.items():
        setattr(dbm, name, timed_call(name, fn))
    for name, m in mods.items():
        def pre(mod, inp, name=name):
            e = torch.cuda.Event(enable_timing=True)
            e.record(stream)
            marks.setdefault(name, []).append([e, None])

        def post(mod, inp, out, name=name):
            e = torch.cuda.Event(enable_timing=True)
            e.record(stream)
            marks[name][-1][1] = e
        handles += [m.register_forward_pre_hook(pre), m.register_forward_hook(post)]
    b0, b1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    b0.record(stream)
    for _ in range(steps):
        step()
    b1.record(stream)
    torch.cuda.synchronize()
    for h in handles:
        h.remove()
    for name, fn in wrapped.items():
        setattr(dbm, name, fn)
    per = {k: sum(a.elapsed_time(b) for a, b in v) / steps for k, v in marks.items()}
    for k in list(mods) + list(wrapped):  # parts the fused path does not call
        per.setdefault(k, 0.0)
    # The attention kernel alone on the block's own inputs and routing: with
    # V as the block passes it (a strided view of the QKV output, token
    # stride 3 H D) and with V copied head-major.
    alone = None
    if "bsa_attention" in seen:
        import math as _m

        from lcv_bsa import _lib
        from lcv_bsa.block_sparse_attention import _geom, _strides
        from lcv_bsa.block_sparse_attention_hip import schedule_block_order
        (q_, k_, v_, shape_), kw_, (_, idx_) = seen["bsa_attention"]
        order_ = schedule_block_order(idx_)
        v_c = v_.contiguous()
        o_ = torch.empty_like(q_)
        lib = _lib.load()
        code = {torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}[q_.dtype]
        geom = _geom(shape_, kw_["chunk_thw"])
        Bq, Hq, Sq, Dq = q_.shape

        def attn_alone(vv):
            _lib.check(lib.lcv_bsa_attn_fwd(
                q_.data_ptr(), k_.data_ptr(), vv.data_ptr(), code, Bq, Hq, Sq, Dq, _strides(q_), _strides(k_),
                _strides(vv), idx_.data_ptr(), order_.data_ptr(), idx_.shape[3], kw_["sm_scale"], geom,
                o_.data_ptr(), _strides(o_), stream.cuda_stream), "attn")

        def timed_alone(vv, n):
            for _ in range(2):
                attn_alone(vv)
            a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a0.record(stream)
            for _ in range(n):
                attn_alone(vv)
            a1.record(stream)
            torch.cuda.synchronize()
            return a0.elapsed_time(a1) / n
        n_alone = max(3, steps)
        alone = {"v_strided_ms": round(timed_alone(v_, n_alone), 3),
                 "v_contiguous_ms": round(timed_alone(v_c, n_alone), 3),
                 "v_strides": list(v_.stride())}
        del q_, k_, v_, v_c, o_, idx_, order_
    seen.clear()
    ms_instr = b0.elapsed_time(b1) / steps
    bsa_ms = per["self_attn"] - per["qkv_gemm"] - per["proj_gemm"]
    Hf = blk.ffn.hidden_dim
    gemm_flop = 2 * N * C * (3 * C + C + C + C + 3 * Hf) + 2 * L * C * 2 * C
    ffn_ms = per["ffn"]
    other = ms_instr - per["self_attn"] - per["cross_attn"] - per["pre_cross_norm"] - ffn_ms
    del blk, x, y, t
    torch.cuda.empty_cache()
    name = DTYPE_NAME[str(dt).split(".")[1]]
    return {
        "workload": "one LongCat-Video DiT block, 720p refinement latents (16, 45, 80) = 57600 tokens, hidden 4096, "
                    f"32 heads x 128, SwiGLU 11008, 512 text tokens, {name} activations, random weights",
        "dtype": name,
        "bsa": f"fused prepare_qk + BSA, 64-token blocks, top-k {top_k} of 900",
        "ms": round(ms, 3),
        "bsa_ms": round(bsa_ms, 3),
        "bsa_share": round(bsa_ms / ms_instr, 4),
        "bsa_parts_ms": {
            "prepare_qk": round(per["prepare_qk"], 3),
            "bsa_attention (routing + launch order + attention)": round(per["bsa_attention"], 3),
            "between (host work with the GPU idle)": round(bsa_ms - per["prepare_qk"] - per["bsa_attention"], 3),
        },
        "attention_alone_on_block_inputs": alone,
        "breakdown_ms": {
            "self_attn_qkv_gemm": round(per["qkv_gemm"], 3),
            "self_attn_bsa (prepare_qk + routing + attention)": round(bsa_ms, 3),
            "self_attn_proj_gemm": round(per["proj_gemm"], 3),
            "cross_attn (q/kv/proj GEMMs, q/k norms, attention over 512 text tokens)":
                round(per["cross_attn"] + per["pre_cross_norm"], 3),
            "ffn (w1|w3 and w2 GEMMs + SiLU gate)": round(ffn_ms, 3),
            "adaln_modulation_residuals_and_pre_norm": round(other, 3),
        },
        "gemm_tflop": round(gemm_flop / 1e12, 3),
        "instrumented_ms": round(ms_instr, 3),
    }


def bench_kv_split(lib, dev, stream, steps: int, warmup: int, seed: int):
    """BSA where queries and keys differ in length: the noise queries of a
    720p continuation (16 noise latent frames after 4 conditioning frames)
    over all 20 frames' keys -- the case the reference sends to dense
    attention (attention.py:218-221).  B=1, 32 heads, D=128, fp16, 64-token
    blocks: nq = 900 q-blocks over nk = 1125 k-blocks, top-k 71
    (ceil(0.0625 * 1125)).  Synthetic inputs as the headline workload's, with
    RoPE on the full (20, 45, 80) grid."""
    import torch

    from lcv_bsa import _lib
    from lcv_bsa.block_sparse_attention import (
        _geom, _strides, bsa_attention, mean_pool_blocks_3d, select_block_indices,
    )
    from lcv_bsa.block_sparse_attention_hip import schedule_block_order
    from lcv_bsa.workloads import make_inputs

    grid, ncl, H, D, top_k = (20, 45, 80), 4, 32, 128, 71
    Sk = grid[0] * grid[1] * grid[2]
    nc = ncl * grid[1] * grid[2]
    Sq = Sk - nc
    q_all, k, v, _ = make_inputs(1, H, D, (1, 1, Sk), (1, 1, 64), torch.float16, dev, seed=seed + 4, grid=grid)
    q = q_all[:, :, nc:]
    qshape, kshape, chunk = (1, 1, Sq), (1, 1, Sk), (1, 1, 64)
    idx = select_block_indices(mean_pool_blocks_3d(q, qshape, chunk), mean_pool_blocks_3d(k, kshape, chunk), top_k)
    order = schedule_block_order(idx, Sk // 64)
    out = torch.empty_like(q)
    sh = stream.cuda_stream
    scale = 1.0 / math.sqrt(D)

    def attn():
        _lib.check(lib.lcv_bsa_attn_fwd_kv(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.F16, 1, H, Sq, Sk, D, _strides(q), _strides(k),
            _strides(v), idx.data_ptr(), order.data_ptr(), top_k, scale, _geom(qshape, chunk), _geom(kshape, chunk),
            out.data_ptr(), _strides(out), sh), "attn_fwd_kv")

    def full():
        bsa_attention(q, k, v, qshape, chunk_thw=chunk, sm_scale=scale, top_k=top_k, kv_shape=kshape)

    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / n

    for _ in range(warmup):
        attn()
        full()
    ms_attn = timed(attn, steps)
    ms_full = timed(full, steps)
    from torch.nn.attention import SDPBackend, sdpa_kernel

    def dense():
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=scale)
    try:
        dense()
        ms_dense = timed(dense, 2)
    except RuntimeError as e:  # no fused SDPA kernel for this shape
        log(f"dense SDPA unavailable: {e}")
        ms_dense = None
    flop = 4 * H * (Sq // 64) * top_k * 64 * 64 * D
    tflops = flop / (ms_attn * 1e-3) / 1e12
    del q_all, k, v, out
    torch.cuda.empty_cache()
    return {
        "workload": "720p continuation: noise queries (16 latent frames, 57600 tokens) over 4 conditioning + 16 "
                    "noise frames of keys (72000 tokens), B1 H32 D128 fp16, 64-token blocks, top-k 71 of 1125",
        "ms_attention": round(ms_attn, 4),
        "executed_tflop": round(flop / 1e12, 4),
        "achieved": round(tflops, 1),
        "frac_of_2500": round(tflops / 2500.0, 4),
        "ms_total": round(ms_full, 4),
        "dense_sdpa_ms": None if ms_dense is None else round(ms_dense, 3),
    }


def bench_voxel_policy(lib, dev, stream, steps: int, warmup: int, seed: int):
    """The block-geometry choice at a 720p-sized grid that the (4, 4, 4)
    voxel can tile: (16, 48, 80) latents (720p padded from 45 to 48 rows),
    B1 H32 D128 fp16, top-k 60 of 960 blocks.  The same q, k, v go through
    the attention kernel once with (4, 4, 4) voxel blocks and once with
    64-token runs, each with its own top-k routing."""
    import torch

    from lcv_bsa import _lib
    from lcv_bsa.block_sparse_attention import _geom, _strides, mean_pool_blocks_3d, select_block_indices
    from lcv_bsa.block_sparse_attention_hip import schedule_block_order
    from lcv_bsa.workloads import make_inputs

    grid, H, D, top_k = (16, 48, 80), 32, 128, 60
    S = grid[0] * grid[1] * grid[2]
    q, k, v, _ = make_inputs(1, H, D, grid, (4, 4, 4), torch.float16, dev, seed=seed + 5, grid=grid)
    out = torch.empty_like(q)
    sh = stream.cuda_stream
    res = {}
    for name, shape, chunk in (("voxel_4x4x4", grid, (4, 4, 4)), ("contiguous_64", (1, 1, S), (1, 1, 64))):
        idx = select_block_indices(mean_pool_blocks_3d(q, shape, chunk), mean_pool_blocks_3d(k, shape, chunk), top_k)
        order = schedule_block_order(idx)
        geom = _geom(shape, chunk)

        def attn():
            _lib.check(lib.lcv_bsa_attn_fwd(
                q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.F16, 1, H, S, D, _strides(q), _strides(k),
                _strides(v), idx.data_ptr(), order.data_ptr(), top_k, 1.0 / math.sqrt(D), geom,
                out.data_ptr(), _strides(out), sh), "attn")
        for _ in range(warmup):
            attn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            attn()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        flop = 4 * H * (S // 64) * top_k * 64 * 64 * D
        res[name] = {"ms_attention": round(ms, 4), "achieved": round(flop / (ms * 1e-3) / 1e12, 1)}
    del q, k, v, out
    torch.cuda.empty_cache()
    return {"workload": "latents (16, 48, 80) = 61440 tokens, B1 H32 D128 fp16, top-k 60 of 960, same inputs", **res}


def run_leg(leg: str, lib, w, dev, stream, args, top_k: int) -> int:
    """One secondary leg alone (the headline forward is not run): its JSON
    object on one line."""
    import torch

    if leg == "prepare":
        res = bench_prepare(lib, w, dev, stream, args.steps, args.warmup, args.seed)
    elif leg == "kv_split":
        res = bench_kv_split(lib, dev, stream, args.steps, args.warmup, args.seed)
    elif leg == "block_geometry":
        res = bench_voxel_policy(lib, dev, stream, args.steps, args.warmup, args.seed)
    else:
        dt = torch.float16 if leg == "dit_block" else torch.bfloat16
        res = bench_dit_block(dev, stream, max(3, args.steps // 2), 2, args.seed, top_k, dt)
    print(json.dumps({"leg": leg, **res}), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3"])
    ap.add_argument("--top-k", type=int, default=None)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prepare", action="store_true", help="skip the pre-BSA prepare_qk timing")
    ap.add_argument("--no-dit-block", action="store_true", help="skip the 720p DiT block timing")
    ap.add_argument("--no-kv-split", action="store_true", help="skip the S_q != S_k (continuation) timing")
    ap.add_argument("--leg", default=None,
                    choices=["prepare", "kv_split", "block_geometry", "dit_block", "dit_block_bf16"],
                    help="run only this leg (for profiling it alone) and print its JSON line")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run a device-to-device copy of MIB MiB (a known-size kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    args = ap.parse_args()

    if args.calibrate_copy:
        import torch

        n = args.calibrate_copy * (1 << 20)
        src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n, "launches": 3}))
        return 0

    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                          "(BSA shards by head across GPUs; see the design notes)"}))
        log(f"bench.py: --gpus {args.gpus} requested, but only the single-GPU path exists")
        return 2

    import torch

    from lcv_bsa import _lib
    from lcv_bsa.block_sparse_attention import _geom, _strides
    from lcv_bsa.workloads import CONFIGS, make_workload

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    cfg = CONFIGS[args.config]
    top_k = args.top_k or cfg["top_k"]
    t0 = time.time()
    w = make_workload(args.config, dev, seed=args.seed, top_k=top_k,
                      margin_ks=tuple(sorted({top_k, top_k - 1})))
    torch.cuda.synchronize()
    B, H, S, D = w.q.shape
    nb = w.num_blocks
    dtype = DTYPE_NAME[str(w.q.dtype).split(".")[1]]
    log(f"workload {args.config}: B={B} H={H} S={S} D={D} {dtype} top_k={top_k} nb={nb} "
        f"(margin repairs {w.repairs}, {time.time() - t0:.1f}s)")

    code = {"f16": _lib.F16, "bf16": _lib.BF16, "f32": _lib.F32}[dtype]
    if args.leg is not None:
        return run_leg(args.leg, lib, w, dev, torch.cuda.current_stream(dev), args, top_k)
    out = torch.empty_like(w.q)
    idx = torch.empty((B, H, nb, top_k), dtype=torch.int32, device=dev)
    ws_bytes = lib.lcv_bsa_forward_workspace_bytes(B, H, nb, D)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=dev)
    assert ws.data_ptr() % 256 == 0
    # Workspace layout: qbar, kbar, block scores, launch order (256-byte aligned).
    pooled = (B * H * nb * D * 4 + 255) // 256 * 256
    scored = (B * H * nb * nb * 4 + 255) // 256 * 256
    qbar = ws[:pooled].view(torch.float32)
    kbar = ws[pooled:2 * pooled].view(torch.float32)
    score = ws[2 * pooled:2 * pooled + B * H * nb * nb * 4].view(torch.float32)
    order = ws[2 * pooled + scored:2 * pooled + scored + B * H * nb * 4].view(torch.int32)
    geom = _geom(w.shape, w.chunk_thw)
    qs, ks, vs, os_ = _strides(w.q), _strides(w.k), _strides(w.v), _strides(out)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream

    def forward():
        st = lib.lcv_bsa_forward(w.q.data_ptr(), w.k.data_ptr(), w.v.data_ptr(), code, B, H, S, D,
                                 qs, ks, vs, top_k, w.sm_scale, geom, ws.data_ptr(), ws_bytes,
                                 idx.data_ptr(), out.data_ptr(), os_, sh)
        _lib.check(st, "lcv_bsa_forward")

    def stage_pool():
        _lib.check(lib.lcv_bsa_pool(w.q.data_ptr(), code, B, H, S, D, qs, geom, qbar.data_ptr(), sh), "pool q")
        _lib.check(lib.lcv_bsa_pool(w.k.data_ptr(), code, B, H, S, D, ks, geom, kbar.data_ptr(), sh), "pool k")

    def stage_select():
        _lib.check(lib.lcv_bsa_scores(qbar.data_ptr(), kbar.data_ptr(), B, H, nb, nb, D,
                                      score.data_ptr(), sh), "scores")
        _lib.check(lib.lcv_bsa_topk(score.data_ptr(), B, H, nb, nb, top_k, idx.data_ptr(), sh),
                   "top-k")
        _lib.check(lib.lcv_bsa_schedule(idx.data_ptr(), B, H, nb, top_k, order.data_ptr(), sh),
                   "schedule")

    def stage_attn():
        _lib.check(lib.lcv_bsa_attn_fwd(w.q.data_ptr(), w.k.data_ptr(), w.v.data_ptr(), code, B, H, S,
                                        D, qs, ks, vs, idx.data_ptr(), order.data_ptr(), top_k,
                                        w.sm_scale, geom, out.data_ptr(), os_, sh), "attn")

    for _ in range(args.warmup):
        forward()
    torch.cuda.synchronize()

    # Timed region 1: K full forwards.
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    ev0.record(stream)
    for _ in range(args.steps):
        forward()
    ev1.record(stream)
    torch.cuda.synchronize()
    ms_step = ev0.elapsed_time(ev1) / args.steps

    # The same forwards with an event between each: the median latency of
    # one forward (the timed loop above gives the throughput).
    evf = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    evf[0].record(stream)
    for i in range(args.steps):
        forward()
        evf[i + 1].record(stream)
    torch.cuda.synchronize()
    per_fwd = sorted(evf[i].elapsed_time(evf[i + 1]) for i in range(args.steps))
    ms_median = per_fwd[len(per_fwd) // 2] if len(per_fwd) % 2 else 0.5 * (per_fwd[len(per_fwd) // 2 - 1] + per_fwd[len(per_fwd) // 2])

    # Timed region 2: the same work stage by stage, events between stages.
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
    torch.cuda.synchronize()
    for e in evs:
        e[0].record(stream)
        stage_pool()
        e[1].record(stream)
        stage_select()
        e[2].record(stream)
        stage_attn()
        e[3].record(stream)
    torch.cuda.synchronize()
    ms_pool = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    ms_sel = sum(e[1].elapsed_time(e[2]) for e in evs) / args.steps
    ms_attn = sum(e[2].elapsed_time(e[3]) for e in evs) / args.steps

    flops = w.flops
    tflops = flops / (ms_step * 1e-3) / 1e12
    attn_tflops = flops / (ms_attn * 1e-3) / 1e12
    peak = PEAK_TFLOPS.get(dtype, 2500.0)
    workload = f"{args.config}_k{top_k}"
    log(f"forward {ms_step:.3f} ms (median {ms_median:.3f}; {tflops:.1f} TFLOP/s executed-block); pool {ms_pool:.3f} ms, "
        f"select {ms_sel:.3f} ms, attention {ms_attn:.3f} ms ({attn_tflops:.1f} TFLOP/s, "
        f"{100 * attn_tflops / peak:.1f}% of {peak:.0f})")

    result = {
        "metric": METRIC,
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "ms_forward_median": round(ms_median, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded N(0,1) + per-block low-rank offsets, 3D RoPE 44/42/42, margin-repaired routing)",
        "config": {
            "workload": f"bsa_fwd_{args.config}_B{B}_H{H}_S{S}_D{D}_{dtype}_topk{top_k}",
            "B": B, "H": H, "S": S, "D": D, "num_blocks": nb, "block_tokens": 64,
            "top_k": top_k, "top_k_rule": "ceil(0.0625*nb)" if top_k != max(1, int(0.0625 * nb)) else "floor (reference)",
            "geometry": "shape=(1,1,S), chunk_thw=(1,1,64)",
            "rope_grid": list(w.grid) if w.grid else None,
            "executed_tflop": round(flops / 1e12, 4),
        },
        "breakdown_ms": {"pool": round(ms_pool, 4), "select_and_schedule": round(ms_sel, 4), "attention": round(ms_attn, 4)},
        "roofline": {
            "bound": "mfma",
            "achieved": round(attn_tflops, 2),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(attn_tflops / peak, 4),
            "traffic": _traffic_from_profiles(workload),
        },
        "cpu_baseline": None,
    }
    if w.grid and not args.no_prepare:
        pre = bench_prepare(lib, w, dev, stream, args.steps, args.warmup, args.seed)
        result["pre_bsa"] = pre
        log(f"pre-BSA prepare_qk {pre['ms']:.3f} ms ({pre['achieved']:.0f} GB/s, "
            f"{100 * pre['frac']:.1f}% of HBM, {100 * pre['frac_of_copy']:.1f}% of the box's copy rate "
            f"{pre['copy']['achieved']:.0f} GB/s); unfused torch chain {pre['unfused_torch_ms']:.3f} ms")
    if args.config == "c2" and not args.no_kv_split:
        kv = bench_kv_split(lib, dev, stream, args.steps, args.warmup, args.seed)
        result["kv_split"] = kv
        log(f"S_q != S_k (continuation): attention {kv['ms_attention']:.3f} ms ({kv['achieved']:.0f} TFLOP/s, "
            f"{100 * kv['frac_of_2500']:.1f} %), pipeline {kv['ms_total']:.3f} ms; dense SDPA {kv['dense_sdpa_ms']} ms")
    if args.config == "c2" and not args.no_kv_split:
        vp = bench_voxel_policy(lib, dev, stream, args.steps, args.warmup, args.seed)
        result["block_geometry"] = vp
        log(f"geometry at (16,48,80): voxel {vp['voxel_4x4x4']['ms_attention']:.3f} ms, "
            f"contiguous {vp['contiguous_64']['ms_attention']:.3f} ms")
    if args.config == "c2" and not args.no_dit_block:
        for key, dt in (("dit_block", torch.float16), ("dit_block_bf16", torch.bfloat16)):
            blk = bench_dit_block(dev, stream, max(3, args.steps // 2), 2, args.seed, top_k, dt)
            result[key] = blk
            log(f"DiT block 720p {blk['dtype']}: {blk['ms']:.2f} ms, BSA {blk['bsa_ms']:.2f} ms = "
                f"{100 * blk['bsa_share']:.1f} % ({blk['breakdown_ms']})")
    if not args.no_cpu_baseline:
        t0 = time.time()
        result["cpu_baseline"] = cpu_baseline(w, args.cpu_budget)
        log(f"cpu baseline: {result['cpu_baseline']['value'] * 1e3:.2f} GFLOP/s ({time.time() - t0:.1f}s)")
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
