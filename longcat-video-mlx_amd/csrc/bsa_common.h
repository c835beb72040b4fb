// Shared device/host helpers for the gfx950 block sparse attention kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lcv_bsa.h"

namespace lcv {

// ---------------------------------------------------------------------------
// Element types.  The kernels move raw 16-bit patterns; arithmetic happens in
// fp32 (VALU) or on MFMA with fp32 accumulation.
// ---------------------------------------------------------------------------
typedef _Float16 f16;
typedef __bf16 bf16;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float to_f32(f16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
__device__ __forceinline__ float to_f32(float x) { return x; }

template <typename T>
__device__ __forceinline__ T from_f32(float x);
template <>
__device__ __forceinline__ f16 from_f32<f16>(float x) { return (f16)x; }
template <>
__device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }
template <>
__device__ __forceinline__ float from_f32<float>(float x) { return x; }

// Bits of a 16-bit element in the low half of a u32.
template <typename T>
__device__ __forceinline__ uint32_t bits16(T x) {
  return (uint32_t)__builtin_bit_cast(uint16_t, x);
}

// ---------------------------------------------------------------------------
// Block geometry: block n of a (T, Hl, Wl) grid cut into (cT, cH, cW) voxels.
// Token index of row r of block n (rows ordered (i, j, l) over the voxel):
//   s = (bt*cT + i)*Hl*Wl + (bh*cH + j)*Wl + bw*cW + l.
// ---------------------------------------------------------------------------
struct Geom {
  int32_t Hl, Wl;      // grid rows / columns per frame
  int32_t cT, cH, cW;  // voxel
  int32_t Bh, Bw;      // blocks per grid column axis / row axis
  int32_t HW;          // Hl * Wl
};

__host__ inline Geom make_geom(const lcv_bsa_geom& g) {
  Geom r;
  r.Hl = (int32_t)g.Hl;
  r.Wl = (int32_t)g.Wl;
  r.cT = (int32_t)g.cT;
  r.cH = (int32_t)g.cH;
  r.cW = (int32_t)g.cW;
  r.Bh = (int32_t)(g.Hl / g.cH);
  r.Bw = (int32_t)(g.Wl / g.cW);
  r.HW = (int32_t)(g.Hl * g.Wl);
  return r;
}

// First token of block n.
__device__ __forceinline__ int32_t block_base_token(const Geom& g, int32_t n) {
  const int32_t per_t = g.Bh * g.Bw;
  const int32_t bt = n / per_t;
  const int32_t rem = n - bt * per_t;
  const int32_t bh = rem / g.Bw;
  const int32_t bw = rem - bh * g.Bw;
  return bt * g.cT * g.HW + bh * g.cH * g.Wl + bw * g.cW;
}

// Division by a run-time invariant divisor with a multiply-high, exact for
// every 32-bit unsigned numerator (Granlund & Montgomery, "Division by
// Invariant Integers using Multiplication", PLDI 1994, figure 4.1):
//   l = ceil(log2 d), m = floor(2^32 (2^l - d) / d) + 1,
//   t = mulhi(m, n),  n / d = (t + ((n - t) >> min(l, 1))) >> max(l - 1, 0).
struct FastDiv {
  uint32_t d, m, s1, s2;
};

__host__ inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((uint64_t{1} << l) < d) ++l;
  FastDiv f;
  f.d = d;
  f.m = (uint32_t)(((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1);
  f.s1 = l > 0 ? 1u : 0u;
  f.s2 = l > 0 ? l - 1 : 0u;
  return f;
}

__device__ __forceinline__ uint32_t fast_div(uint32_t n, const FastDiv& f) {
  const uint32_t t = __umulhi(f.m, n);
  return (t + ((n - t) >> f.s1)) >> f.s2;
}

// Token offset of row r inside any block, relative to the block's first token.
__device__ __forceinline__ int32_t voxel_row_offset(const Geom& g, int32_t r) {
  const int32_t plane = g.cH * g.cW;
  const int32_t i = r / plane;
  const int32_t rem = r - i * plane;
  const int32_t j = rem / g.cW;
  const int32_t l = rem - j * g.cW;
  return i * g.HW + j * g.Wl + l;
}

// ---------------------------------------------------------------------------
// Work-item order that keeps each XCD on few heads.  Workgroups are handed to
// the 8 XCDs of an MI355X round robin (XCD = blockIdx % 8).  This maps
// blockIdx to a linear work id so that XCD x processes a contiguous range of
// work ids; consecutive work ids are the q-blocks of one head, so the K/V
// blocks that the concurrently resident workgroups of an XCD read come from
// one head and are re-served from that XCD's L2.
// ---------------------------------------------------------------------------
constexpr int kNumXcd = 8;

__device__ __forceinline__ int32_t xcd_linear_work_id(int32_t bid, int32_t total) {
  const int32_t xcd = bid % kNumXcd;
  const int32_t slot = bid / kNumXcd;
  const int32_t base = total / kNumXcd;
  const int32_t extra = total % kNumXcd;
  const int32_t start = xcd * base + (xcd < extra ? xcd : extra);
  return start + slot;
}

// ---------------------------------------------------------------------------
// Wave helpers (wave64).
// ---------------------------------------------------------------------------
__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t mbcnt64(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

__device__ __forceinline__ uint64_t ballot64(bool p) { return __ballot(p); }

__device__ __forceinline__ int32_t uniform_i32(int32_t x) {
  return __builtin_amdgcn_readfirstlane(x);
}

}  // namespace lcv

// ---------------------------------------------------------------------------
// Host-side launchers implemented in the kernel translation units.  Each
// returns a hipError_t; argument validation happens in capi.cpp.
// ---------------------------------------------------------------------------
namespace lcv {

struct Tensor4 {
  const void* ptr;
  int64_t sb, sh, ss;  // element strides; D axis dense
};

hipError_t launch_pool(const Tensor4* xs, int n_tensors, int dtype, int B, int H,
                       int D, int nb, int bs, const Geom& g, float* const* outs,
                       hipStream_t stream);

hipError_t launch_scores(const float* qbar, const float* kbar, int B, int H, int nq,
                         int nk, int D, float* score, hipStream_t stream);
hipError_t launch_topk(const float* score, int B, int H, int nq, int nk, int top_k,
                       int32_t* idx, hipStream_t stream);
hipError_t launch_select(const float* qbar, const float* kbar, int B, int H, int nq,
                         int nk, int D, int top_k, int32_t* idx, hipStream_t stream);
bool select_supported(int nk, int D);

struct AttnParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  const int32_t* idx;     // [B, H, nb, top_k] K/V block ids in [0, nk)
  const int32_t* order;  // [B*H*nb] launch order of q-blocks per head, or null
  int32_t B, H, nb, top_k;  // nb: q-blocks per head
  int32_t nk;               // K/V blocks per head
  float scale_log2;
  // Bytes spanned by one head of k / v (buffer-descriptor extents).
  uint32_t k_head_bytes, v_head_bytes;
  Geom g;   // block geometry of q and out
  Geom gk;  // block geometry of k and v (the same as g unless S_q != S_k)
};

// Chooses the MFMA kernel (fp16/bf16, D in {64,128}, scale >= 0) or the
// vector-ALU kernel (any dtype, D in {16,32,64,128,256}).
hipError_t launch_attn(const AttnParams& p, int dtype, int D, hipStream_t stream);
bool attn_supported(int dtype, int D);
bool attn_uses_mfma(int dtype, int D);

// Per-head q-block launch order from the routing lists (nq <= 4096 q-blocks,
// entries are K/V block ids in [0, nk)).
hipError_t launch_schedule(const int32_t* idx, int BH, int nq, int nk, int top_k, int32_t* order,
                           hipStream_t stream);
bool schedule_supported(int nq, int nk);

// Fused RMSNorm + 3D RoPE + block means of q and k (fp16/bf16, D 64/128).
// The RoPE table holds cos and sin per axis: [rT*dt/2 | rT*dt/2 | rH*dh/2 |
// rH*dh/2 | rW*dw/2 | rW*dw/2] floats, at most kMaxRopeTable.
constexpr int kMaxRopeTable = 12288;
// Token positions are split over the RoPE grid with an fp32 reciprocal, exact
// below 2^22 tokens.
constexpr int64_t kPrepMaxTokens = int64_t{1} << 22;
bool prep_supported(int dtype, int D);
hipError_t launch_prep(const Tensor4* in, const Tensor4* out, const void* const* weight,
                       float* const* mean, int dtype, int B, int H, int D, int nb, const Geom& g,
                       const int32_t* rope_grid, const int32_t* rope_dims, const float* table,
                       int table_len, float eps, hipStream_t stream);

// DiT block row operations (fp16 / bf16).
bool rows_supported(int dtype, int C);
hipError_t launch_rows(const void* x, const void* a, const float* gate, const float* shift,
                       const float* scale, const void* ln_w, const void* ln_b, void* x_out,
                       void* n_out, int dtype, int rows, int C, int rows_per_batch,
                       int tokens_per_frame, int frames, float eps, hipStream_t stream);
hipError_t launch_swiglu(const void* h, void* out, int dtype, int64_t rows, int hidden,
                         hipStream_t stream);
hipError_t launch_head_norm(const void* x, const int64_t* xs, void* out, const int64_t* os,
                            const void* w, int dtype, int B, int N, int H, int D, float eps,
                            hipStream_t stream);

hipError_t launch_token_blocks(const Geom& g, int T, int32_t* out, hipStream_t stream);
hipError_t launch_pair_mask(const int32_t* idx, int B, int H, int nq, int top_k,
                            const int32_t* token_block, int S, int nkv, uint8_t* mask,
                            hipStream_t stream);
hipError_t launch_permute(const void* x, int elem_bytes, int B, int H, int S, int D,
                          const Geom& g, int inverse, void* out, hipStream_t stream);

}  // namespace lcv
