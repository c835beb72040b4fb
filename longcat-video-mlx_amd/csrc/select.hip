// Block routing: block scores qbar . kbar^T of fp32 pooled means and per-row
// top-k.
//
// For head dims 64 and 128 the score GEMM runs on bf16 MFMA with each fp32
// operand split exactly into three bf16 pieces (six piece products, fp32
// accumulation; see below): every product is formed to within 2^-21 of its
// value and the sum is accumulated in fp32, an error of the order of an fp32
// GEMM's.  Other head dims use fp32 FMAs.  Selection is exact given score
// margins well above that rounding.
//
// Follows block_routing_scores + topk_block_indices
// (longcat_video/models/block_sparse_attention.py:107-134).  The reference
// materialises the [B,H,nq,nk] score tensor and runs argpartition; here a
// wave computes whole score rows straight into registers in the layout its
// top-k needs (lane l holds columns l, l+64, l+128, ...), so the fused path
// never writes scores to memory.
//
// Top-k is an exact radix select on order-preserving 32-bit keys: a bit-by-bit
// binary search finds the k-th largest key with ballot/popcount counts (over
// the keys above a cheap exact lower bound, compacted, when k <= 128; only
// the bits below those the bound and the row maximum share), then
// one ordered pass emits the indices of keys above it plus the lowest-index
// keys equal to it, in ascending index order.  Equal scores therefore resolve
// to the lower block index; NaN ranks below -inf; -0.0 equals +0.0.
#include "bsa_common.h"

namespace lcv {
namespace {

constexpr int kMaxD = 128;       // pooled head dim supported by the routing kernels
constexpr int kKeyChunk = 64;    // keys staged per LDS chunk (one per lane)
constexpr int kMaxPer = 64;      // max score columns per lane -> nk <= 4096

__device__ __forceinline__ uint32_t order_key(float f) {
  if (f != f) return 0u;       // NaN: below every number
  if (f == 0.0f) f = 0.0f;     // -0.0 -> +0.0
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

constexpr int kCompactCap = 512;  // compacted keys per wave (LDS words)

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t y = (uint32_t)__shfl_xor((int)x, o);
    x = y < x ? y : x;
  }
  return x;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t y = (uint32_t)__shfl_xor((int)x, o);
    x = y > x ? y : x;
  }
  return x;
}

// Largest t with #(key >= t) >= k, built bit by bit over R keys per lane
// (padding keys are 0 and never reach a candidate >= 1).  `floor` is at most
// the k-th largest key (#(key >= floor) >= k) and `hi` at least every key, so
// the k-th largest key lies in [floor, hi] and carries the bits that floor
// and hi share above their highest differing bit: the search starts with
// those bits set as in floor (the bit-by-bit search from bit 31 would set
// exactly them) and decides only the bits below.  Once a candidate at or
// above `floor` has exactly k keys at or above it, those keys are the top k
// and the remaining bits cannot change the selection.
template <int R>
__device__ uint32_t kth_key(const uint32_t (&key)[R], int k, uint32_t floor, uint32_t hi) {
  const uint32_t diff = floor ^ hi;
  if (diff == 0u) return floor;  // every key from floor to hi equals floor
  const int top = 31 - __builtin_clz(diff);
  uint32_t thr = floor & ~(uint32_t)((2ull << top) - 1ull);
  for (int bit = top; bit >= 0; --bit) {
    const uint32_t cand = thr | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) cnt += __popcll(ballot64(key[r] >= cand));
    if (cnt >= k) {
      thr = cand;
      if (cnt == k && cand >= floor) break;
    }
  }
  return thr;
}


// Emits, in ascending column order, the k selected entries among R keys per
// lane at list positions lane + 64 r (r < R; positions >= n are not keys):
// those above thr, then the lowest-positioned ones equal to it.  Positions
// must follow ascending column order; col(r) gives the column of register r.
template <int R, typename ColFn>
__device__ __forceinline__ void emit_selected(const uint32_t (&key)[R], int n, uint32_t thr, int k,
                                              int32_t* out, ColFn col) {
  const int lane = lane_id();
  int gt = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) gt += __popcll(ballot64(lane + 64 * r < n && key[r] > thr));
  const int need_eq = k - gt;
  int run_sel = 0, run_eq = 0;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const bool valid = lane + 64 * r < n;
    const bool is_gt = valid && key[r] > thr;
    const bool is_eq = valid && key[r] == thr;
    const uint64_t eqm = ballot64(is_eq);
    const int eq_rank = run_eq + (int)mbcnt64(eqm);
    const bool sel = is_gt || (is_eq && eq_rank < need_eq);
    const uint64_t selm = ballot64(sel);
    if (sel) out[run_sel + (int)mbcnt64(selm)] = col(r);
    run_sel += __popcll(selm);
    run_eq += __popcll(eqm);
  }
}

// Compacted keys a wave keeps for a row of NPER keys per lane.
template <int NPER>
constexpr int compact_cap() { return NPER * 64 < kCompactCap ? NPER * 64 : kCompactCap; }

// Exact top-k of one score row held as sc[e] = score[e*64 + lane], e < NPER.
// Writes the k selected column indices, ascending, to out[0..k).  buf:
// 2 compact_cap<NPER>() words of this wave's LDS (keys, then their columns).
//
// For k <= 64 (and nk >= 64) a lower bound on the k-th largest key comes
// first: every lane's largest key is >= L = their minimum, so at least
// 64 >= k keys are >= L and the k-th largest key is among the keys >= L.
// For 64 < k <= 128 (and nk >= 128) the lanes' second-largest keys give the
// bound the same way (at least 128 keys are >= their minimum).  The keys
// >= L (typically a quarter or a third of the row) are compacted, in column
// order, with their columns, into 4 or 8 registers per lane; the search and
// the emission then run over them only (counts at candidates >= L equal the
// full row's, below L both are >= k, so the threshold is the full row's).
template <int NPER>
__device__ void wave_topk(const float (&sc)[NPER], int nk, int k, int32_t* out, uint32_t* buf) {
  const int lane = lane_id();
  uint32_t key[NPER];
#pragma unroll
  for (int e = 0; e < NPER; ++e) {
    const int col = e * 64 + lane;
    key[e] = col < nk ? order_key(sc[e]) : 0u;
  }
  constexpr int CAP = compact_cap<NPER>();
  if ((k <= 64 && nk >= 64) || (k <= 128 && nk >= 128)) {  // wave-uniform
    uint32_t m = 0u;   // this lane's largest key (k <= 64) or second-largest key
    uint32_t m1 = 0u;  // this lane's largest key
    if (k <= 64) {
#pragma unroll
      for (int e = 0; e < NPER; ++e) m = key[e] > m ? key[e] : m;
      m1 = m;
    } else {
#pragma unroll
      for (int e = 0; e < NPER; ++e) {
        const uint32_t lo = key[e] < m1 ? key[e] : m1;
        m = lo > m ? lo : m;
        m1 = key[e] > m1 ? key[e] : m1;
      }
    }
    const uint32_t L = wave_min_u32(m);
    const uint32_t hi = wave_max_u32(m1);  // the row's largest key
    int total = 0;
#pragma unroll
    for (int e = 0; e < NPER; ++e) {
      const bool in = e * 64 + lane < nk && key[e] >= L;
      const uint64_t msk = ballot64(in);
      const int pos = total + (int)mbcnt64(msk);
      if (in && pos < CAP) {
        buf[pos] = key[e];
        buf[CAP + pos] = (uint32_t)(e * 64 + lane);
      }
      total += __popcll(msk);
    }
    if (total <= 256) {
      uint32_t ck[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) ck[r] = lane + 64 * r < total ? buf[lane + 64 * r] : 0u;
      const uint32_t thr = kth_key<4>(ck, k, L, hi);
      emit_selected<4>(ck, total, thr, k, out, [&](int r) { return (int32_t)buf[CAP + lane + 64 * r]; });
      return;
    }
    if (total <= CAP) {
      uint32_t ck[8];
#pragma unroll
      for (int r = 0; r < 8; ++r) ck[r] = lane + 64 * r < total ? buf[lane + 64 * r] : 0u;
      const uint32_t thr = kth_key<8>(ck, k, L, hi);
      emit_selected<8>(ck, total, thr, k, out, [&](int r) { return (int32_t)buf[CAP + lane + 64 * r]; });
      return;
    }
  }
  const uint32_t thr = kth_key<NPER>(key, k, 0u, 0xffffffffu);
  emit_selected<NPER>(key, nk, thr, k, out, [&](int r) { return (int32_t)(r * 64 + lane); });
}

struct RouteArgs {
  const float* qbar;
  const float* kbar;
  const float* score_in;
  float* score_out;
  int32_t* idx;
  int32_t H, nq, nk, D, top_k;
  int32_t tiles_per_bh;
  int32_t col_splits;
};

enum RouteMode { kSelect = 0, kScoresOnly = 1, kTopkOnly = 2 };

// One workgroup = 4 waves x RW score rows of one (b, h).  Lane l of a wave
// owns score columns e*64 + l; the 64 kbar rows of chunk e are staged in LDS
// (row stride D+4 floats: conflict-free 16-byte reads), the workgroup's qbar
// rows are read as LDS broadcasts.
template <int NPER, int RW, int MODE>
__global__ __launch_bounds__(256) void route_kernel(RouteArgs a) {
  __shared__ __attribute__((aligned(16))) float kch[kKeyChunk * (kMaxD + 4)];
  __shared__ __attribute__((aligned(16))) float qt[4 * RW * kMaxD];
  __shared__ uint32_t tk_buf[4][2 * kCompactCap];
  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int bh = blockIdx.x / a.tiles_per_bh;
  const int tile = blockIdx.x - bh * a.tiles_per_bh;
  const int row0 = tile * (4 * RW) + wave * RW;  // this wave's first row
  const int D = a.D;
  const int KS = D + 4;
  float sc[RW][NPER];

  if (MODE == kTopkOnly) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int row = row0 + r;
      const float* src = a.score_in + ((int64_t)bh * a.nq + (row < a.nq ? row : 0)) * a.nk;
#pragma unroll
      for (int e = 0; e < NPER; ++e) {
        const int col = e * 64 + lane;
        sc[r][e] = (row < a.nq && col < a.nk) ? src[col] : 0.0f;
      }
    }
  } else {
    const float* qb = a.qbar + (int64_t)bh * a.nq * D;
    const float* kb = a.kbar + (int64_t)bh * a.nk * D;
    const int D4 = D / 4;
    const int wg_row0 = tile * (4 * RW);
    for (int i = tid; i < 4 * RW * D4; i += 256) {
      const int r = i / D4;
      const int c = i - r * D4;
      const int row = wg_row0 + r;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (row < a.nq) v = *reinterpret_cast<const f32x4*>(qb + (int64_t)row * D + 4 * c);
      *reinterpret_cast<f32x4*>(qt + r * D + 4 * c) = v;
    }
#pragma unroll
    for (int e = 0; e < NPER; ++e) {
      __syncthreads();  // previous chunk fully consumed; qt visible
      for (int i = tid; i < kKeyChunk * D4; i += 256) {
        const int kr = i / D4;
        const int c = i - kr * D4;
        const int key = e * kKeyChunk + kr;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (key < a.nk) v = *reinterpret_cast<const f32x4*>(kb + (int64_t)key * D + 4 * c);
        *reinterpret_cast<f32x4*>(kch + kr * KS + 4 * c) = v;
      }
      __syncthreads();
      float acc[RW];
#pragma unroll
      for (int r = 0; r < RW; ++r) acc[r] = 0.0f;
      const float* krow = kch + lane * KS;
      for (int d = 0; d < D; d += 4) {
        const f32x4 kv = *reinterpret_cast<const f32x4*>(krow + d);
#pragma unroll
        for (int r = 0; r < RW; ++r) {
          const f32x4 qv = *reinterpret_cast<const f32x4*>(qt + (wave * RW + r) * D + d);
          acc[r] = fmaf(qv[0], kv[0], acc[r]);
          acc[r] = fmaf(qv[1], kv[1], acc[r]);
          acc[r] = fmaf(qv[2], kv[2], acc[r]);
          acc[r] = fmaf(qv[3], kv[3], acc[r]);
        }
      }
#pragma unroll
      for (int r = 0; r < RW; ++r) sc[r][e] = acc[r];
    }
  }

  if (MODE == kScoresOnly) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int row = row0 + r;
      if (row >= a.nq) continue;
      float* dst = a.score_out + ((int64_t)bh * a.nq + row) * a.nk;
#pragma unroll
      for (int e = 0; e < NPER; ++e) {
        const int col = e * 64 + lane;
        if (col < a.nk) dst[col] = sc[r][e];
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int row = row0 + r;
      if (row >= a.nq) continue;  // wave-uniform
      wave_topk<NPER>(sc[r], a.nk, a.top_k, a.idx + ((int64_t)bh * a.nq + row) * a.top_k,
                      tk_buf[wave]);
    }
  }
}

// ---------------------------------------------------------------------------
// Score GEMM for head dims 64 and 128 on bf16 MFMA (v_mfma_f32_32x32x16_bf16)
// with fp32 operands split exactly into three bf16 pieces.
//
// A finite fp32 x has 24 significand bits; p0 = x with the low 16 bits of its
// encoding cleared (the top 8 significand bits), p1 the same truncation of
// x - p0, and p2 = x - p0 - p1 (at most 8 significand bits, exactly a bf16).
// Every subtraction is exact, so x = p0 + p1 + p2.  A product x y is formed
// from the six piece products p_i q_j with i + j <= 2; each is exact in fp32
// (8 x 8 bits), and the three dropped ones (i + j >= 3) are below
// 2^-21 |x y| together.  The MFMAs accumulate the six products of every
// 16-dim k-step into one fp32 accumulator, k-steps ascending, in the order
// p0q0, p0q1, p1q0, p0q2, p1q1, p2q0.  Both kernels below issue that MFMA
// sequence per score with the same lane layout (lane (c, g) of a 32 x 16
// operand holds dims 16s + 8g .. + 8 of row c), so they produce identical
// scores.  An inf or NaN goes whole into p0; its product with the other
// operand's p0 carries it as an fp32 product would, and the cross products
// take p0 without it (tile_step_nf), so non-finite scores come out as the
// fp32 GEMM's do.
// ---------------------------------------------------------------------------

// Pieces of 8 consecutive fp32 values, as three bf16x8 operands.  Finite
// values only (the callers route blocks holding inf / NaN to split8_any).
__device__ __forceinline__ void split8(const f32x4& lo, const f32x4& hi, bf16x8 (&pc)[3]) {
  uint32_t w[3][4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    uint32_t u[2], u1[2], u2[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const float x = h < 2 ? lo[2 * h + e] : hi[2 * h - 4 + e];
      u[e] = __builtin_bit_cast(uint32_t, x);
      const float r1 = x - __builtin_bit_cast(float, u[e] & 0xffff0000u);
      u1[e] = __builtin_bit_cast(uint32_t, r1);
      const float r2 = r1 - __builtin_bit_cast(float, u1[e] & 0xffff0000u);
      u2[e] = __builtin_bit_cast(uint32_t, r2);
    }
    // High halves of the pair: element 2h in the low 16 bits.
    w[0][h] = __builtin_amdgcn_perm(u[1], u[0], 0x07060302u);
    w[1][h] = __builtin_amdgcn_perm(u1[1], u1[0], 0x07060302u);
    w[2][h] = __builtin_amdgcn_perm(u2[1], u2[0], 0x07060302u);
  }
#pragma unroll
  for (int q = 0; q < 3; ++q)
    pc[q] = __builtin_bit_cast(bf16x8, (u32x4){w[q][0], w[q][1], w[q][2], w[q][3]});
}

// Any fp32 values: inf and NaN go whole into piece 0 (a NaN stays a NaN in
// its bf16 high half) with pieces 1 and 2 zero; finite values as split8.
__device__ __forceinline__ void split8_any(const f32x4& lo, const f32x4& hi, bf16x8 (&pc)[3]) {
  f32x4 a = lo, b = hi;
  uint32_t fix[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float x = e < 4 ? a[e] : b[e - 4];
    const uint32_t u = __builtin_bit_cast(uint32_t, x);
    const bool fin = (u & 0x7f800000u) != 0x7f800000u;
    // Piece 0 of a non-finite value: its own bits, quiet bit set for a NaN.
    fix[e] = fin ? 0u : (u | ((u & 0x007fffffu) ? 0x00400000u : 0u));
    if (e < 4) a[e] = fin ? x : 0.0f; else b[e - 4] = fin ? x : 0.0f;
  }
  split8(a, b, pc);
  uint32_t w0[4];
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const uint32_t f = __builtin_amdgcn_perm(fix[2 * h + 1], fix[2 * h], 0x07060302u);
    w0[h] = f;
  }
  u32x4 p0 = __builtin_bit_cast(u32x4, pc[0]);
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    // Replace the 16-bit halves whose value was non-finite.
    const uint32_t mlo = fix[2 * h] ? 0x0000ffffu : 0u;
    const uint32_t mhi = fix[2 * h + 1] ? 0xffff0000u : 0u;
    p0[h] = (p0[h] & ~(mlo | mhi)) | (w0[h] & (mlo | mhi));
  }
  pc[0] = __builtin_bit_cast(bf16x8, p0);
}

// Bits of element i of a float vector.  The element goes through a scalar
// first: this compiler bit-casts a vector element subscript passed straight
// to __builtin_bit_cast as element 0.
__device__ __forceinline__ uint32_t elem_bits(const f32x4& v, int i) {
  const float f = v[i];
  return __builtin_bit_cast(uint32_t, f);
}

// True when none of the 8 values is inf / NaN.
__device__ __forceinline__ bool all_finite8(const f32x4& lo, const f32x4& hi) {
  uint32_t m = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    m |= ((elem_bits(lo, e) & 0x7f800000u) == 0x7f800000u) ? 1u : 0u;
    m |= ((elem_bits(hi, e) & 0x7f800000u) == 0x7f800000u) ? 1u : 0u;
  }
  return m == 0;
}

// Pieces of 8 fp32 values, finite or not (wave-uniform choice of path).
__device__ __forceinline__ void split8_wave(const f32x4& lo, const f32x4& hi, bf16x8 (&pc)[3]) {
  if (__ballot(!all_finite8(lo, hi)))
    split8_any(lo, hi, pc);
  else
    split8(lo, hi, pc);
}

// One k-step (16 dims) of a 32 x 32 score tile on v_mfma_f32_32x32x16_bf16:
// the six piece products in a fixed order (p0 q0, p0 q1, p1 q0, p0 q2, p1 q1,
// p2 q0) into one fp32 accumulator.
__device__ __forceinline__ void tile_step(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x16& acc) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
}

// tile_step on two key tiles sharing the A pieces, the two accumulator
// chains interleaved (each chain keeps tile_step's product order).
__device__ __forceinline__ void tile_step2(const bf16x8 (&a)[3], const bf16x8 (&b)[3], const bf16x8 (&c)[3],
                                           f32x16& acc, f32x16& acd) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
  acd = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], c[0], acd, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  acd = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], c[1], acd, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  acd = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], c[0], acd, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
  acd = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], c[2], acd, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acd = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], c[1], acd, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
  acd = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], c[0], acd, 0, 0, 0);
}

// Piece 0 with its inf / NaN halves (bf16 exponent all ones) set to zero.
__device__ __forceinline__ bf16x8 finite_part(const bf16x8& v) {
  u32x4 w = __builtin_bit_cast(u32x4, v);
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const uint32_t m = w[h] & 0x7f807f80u;
    if ((m & 0xffffu) == 0x7f80u) w[h] &= 0xffff0000u;
    if ((m >> 16) == 0x7f80u) w[h] &= 0x0000ffffu;
  }
  return __builtin_bit_cast(bf16x8, w);
}

// tile_step for operands that may hold inf / NaN (in piece 0; pieces 1 and 2
// of such values are zero).  The product of the two pieces 0 carries them as
// an fp32 product would; the cross products take piece 0 without them, so
// no inf meets a zero piece of the other operand.  For finite operands the
// values, and so the result, are those of tile_step.
__device__ __forceinline__ void tile_step_nf(const bf16x8 (&a)[3], const bf16x8 (&b)[3], f32x16& acc) {
  // Opaque copies: the finite parts are formed here, on this rare path, and
  // not hoisted next to the operands they come from (they would hold
  // registers for the whole kernel).
  bf16x8 a0 = a[0], b0 = b[0];
  asm volatile("" : "+v"(a0), "+v"(b0));
  a0 = finite_part(a0);
  b0 = finite_part(b0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b0, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b0, acc, 0, 0, 0);
}

// The A pieces of 32 rows (row0 + lane % 32) for all k-steps: lane (r, g)
// holds dims 16s + 8g .. + 8 of its row.  Rows at or past `nrows` (and
// lanes whose row is not below `live`) are zero.
template <int KST>
__device__ __forceinline__ bool load_row_pieces(const float* base, int row0, int nrows, int D,
                                                int live, bf16x8 (&pa)[KST][3]) {
  const int lane = lane_id();
  const int r = lane % 32;
  const int row = row0 + r;
  const int g = lane / 32;
  bool fin = true;
#pragma unroll
  for (int s = 0; s < KST; ++s) {
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
    if (r < live && row < nrows) {
      const float* src = base + (int64_t)row * D + 16 * s + 8 * g;
      lo = *reinterpret_cast<const f32x4*>(src);
      hi = *reinterpret_cast<const f32x4*>(src + 4);
    }
    fin = fin & all_finite8(lo, hi);
    split8_wave(lo, hi, pa[s]);
  }
  return __ballot(!fin) != 0;
}

// Fused routing for head dims 64 and 128: one workgroup = 16 q-block rows of
// one (b, h) (the top half of a 32-row MFMA block; the bottom half is zero
// and discarded); wave w computes the 32-key score tiles w, w + 4, ..., its
// key operands read from global memory and split in registers.  The 16 x nk
// score rows are gathered in LDS and each wave runs wave_topk on four of
// them: routing without a score buffer.
template <int NPER, int D>
__global__ __launch_bounds__(256) void select_mfma_kernel(RouteArgs a) {
  constexpr int QR = 16;
  constexpr int KST = D / 16;               // k-steps of 16 dims
  constexpr int LDSW = NPER * 64 + 4;       // score row stride (floats)
  // Row stride: the scores, or the top-k buffer the row turns into (2 CAP words).
  constexpr int RSW = LDSW > 2 * compact_cap<NPER>() ? LDSW : 2 * compact_cap<NPER>();
  __shared__ __attribute__((aligned(16))) float srow[QR * RSW];
  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int c = lane % 32;
  const int g = lane / 32;
  const int bh = blockIdx.x / a.tiles_per_bh;
  const int row0 = (blockIdx.x - bh * a.tiles_per_bh) * QR;
  const float* qb = a.qbar + (int64_t)bh * a.nq * D;
  const float* kb = a.kbar + (int64_t)bh * a.nk * D;

  bf16x8 pa[KST][3];
  const bool a_bad = load_row_pieces<KST>(qb, row0, a.nq, D, QR, pa);
  const int ntiles = (a.nk + 31) / 32;
  for (int t = wave; t < ntiles; t += 4) {
    const int key = 32 * t + c;
    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;
    // tile_step_nf equals tile_step on finite operands, so the (wave-uniform)
    // choice can be made per k-step.
#pragma unroll
    for (int s = 0; s < KST; ++s) {
      f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
      if (key < a.nk) {
        const float* src = kb + (int64_t)key * D + 16 * s + 8 * g;
        lo = *reinterpret_cast<const f32x4*>(src);
        hi = *reinterpret_cast<const f32x4*>(src + 4);
      }
      const bool b_bad = __ballot(!all_finite8(lo, hi)) != 0;
      bf16x8 pb[3];
      if (b_bad)
        split8_any(lo, hi, pb);
      else
        split8(lo, hi, pb);
      if (a_bad || b_bad)
        tile_step_nf(pa[s], pb, acc);
      else
        tile_step(pa[s], pb, acc);
    }
    // Rows 8 (i / 4) + 4 g + i % 4 of the tile; i < 8 are the 16 live rows.
#pragma unroll
    for (int i = 0; i < 8; ++i)
      srow[(8 * (i / 4) + 4 * g + i % 4) * RSW + 32 * t + c] = acc[i];
  }
  __syncthreads();
#pragma unroll 1
  for (int r = wave; r < QR; r += 4) {
    const int row = row0 + r;
    if (row >= a.nq) break;  // wave-uniform; rows only grow
    float sc[NPER];
#pragma unroll
    for (int e = 0; e < NPER; ++e) sc[e] = srow[r * RSW + e * 64 + lane];
    // The row's LDS, now in registers, becomes this wave's top-k buffer (LDS
    // operations of one wave complete in order; the fence keeps the
    // compiler from moving the buffer's writes above the row's reads).
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    wave_topk<NPER>(sc, a.nk, a.top_k, a.idx + ((int64_t)bh * a.nq + row) * a.top_k,
                    reinterpret_cast<uint32_t*>(&srow[r * RSW]));
  }
}

// Score matrix S = qbar kbar^T, written to memory.  One workgroup = 4 waves x
// 32 q-block rows (128 rows) of one (b, h) over a range of 64-key chunks
// (col_splits ranges per row tile, so that small heads still fill the GPU).
// Each wave keeps the pieces of its 32 rows in registers.  A chunk's kbar rows
// are read with 16-byte buffer loads (the next chunk's in flight during the
// current chunk's MFMAs; keys past nk read as zero), split, and stored as
// bf16 pieces in LDS (row stride 2D + 16 bytes: the 16-byte operand reads of
// 16 consecutive rows are conflict free); each wave then runs the chunk's two
// 32-key tiles as two interleaved accumulator chains.  Scores go out as
// buffer stores whose offset is pushed out of range for entries past nq or
// nk, so every chunk issues the same memory instructions.
template <int D>
__global__ __launch_bounds__(256) void scores_kernel(RouteArgs a) {
  constexpr int KC = 64;              // keys per chunk
  constexpr int KST = D / 16;         // k-steps of 16 dims
  constexpr int RS = 2 * D + 16;      // LDS row stride of a piece (bytes)
  constexpr int D8 = D / 8;           // 8-value groups per row
  constexpr int kGroups = KC * D8 / 256;
  static_assert(kGroups * 256 == KC * D8, "chunk groups split evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) uint8_t kp[3][KC * RS];
  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int c = lane % 32;
  const int g = lane / 32;
  const int per_bh = a.tiles_per_bh * a.col_splits;
  const int bh = blockIdx.x / per_bh;
  const int rem = blockIdx.x - bh * per_bh;
  const int rt = rem / a.col_splits;
  const int cs = rem - rt * a.col_splits;
  const int row0 = rt * 128 + wave * 32;
  const int nchunks = (a.nk + KC - 1) / KC;
  const int ch0 = (int)((int64_t)cs * nchunks / a.col_splits);
  const int ch1 = (int)((int64_t)(cs + 1) * nchunks / a.col_splits);
  const float* qb = a.qbar + (int64_t)bh * a.nq * D;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.kbar + (int64_t)bh * a.nk * D), (short)0, a.nk * D * 4, 0x00020000);
  // The score resource covers this tile's rows only (at most 128 x 4096
  // scores, 2 MiB), so byte offsets stay far below the drop offset whatever
  // the head's nq x nk.
  const int tile_rows = a.nq - rt * 128 < 128 ? a.nq - rt * 128 : 128;
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(a.score_out + ((int64_t)bh * a.nq + rt * 128) * a.nk), (short)0, tile_rows * a.nk * 4,
      0x00020000);

  bf16x8 pa[KST][3];
  const bool a_bad = load_row_pieces<KST>(qb, row0, a.nq, D, 32, pa);

  // Staging: group i = tid + 256 u of a chunk is key i / D8, dims 8 (i % D8) .. + 8.
  f32x4 st[kGroups][2];
  auto load_chunk = [&](int ch) {
#pragma unroll
    for (int u = 0; u < kGroups; ++u) {
      const int i = tid + 256 * u;
      const uint32_t off = (uint32_t)((ch * KC + i / D8) * D + 8 * (i % D8)) * 4u;
      st[u][0] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
      st[u][1] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, off + 16, 0, 0));
    }
  };
  constexpr uint32_t kDrop = 0x80000000u;  // out-of-range offset: the store is dropped
  if (ch0 < ch1) load_chunk(ch0);
  for (int ch = ch0; ch < ch1; ++ch) {
    __syncthreads();  // the previous chunk is consumed
    bool fin = true;
    {
#pragma unroll
      for (int u = 0; u < kGroups; ++u) fin = fin & all_finite8(st[u][0], st[u][1]);
      const bool any_bad = __ballot(!fin) != 0;  // wave-uniform
#pragma unroll
      for (int u = 0; u < kGroups; ++u) {
        const int i = tid + 256 * u;
        bf16x8 pc[3];
        if (any_bad)
          split8_any(st[u][0], st[u][1], pc);
        else
          split8(st[u][0], st[u][1], pc);
        const int off = (i / D8) * RS + 16 * (i % D8);
#pragma unroll
        for (int q = 0; q < 3; ++q) *reinterpret_cast<bf16x8*>(&kp[q][off]) = pc[q];
      }
    }
    // Barrier (every thread reaches it); true when any thread staged an inf / NaN.
    const bool chunk_bad = __syncthreads_or(!fin) != 0;
    const bool bad = a_bad || chunk_bad;
    if (ch + 1 < ch1) load_chunk(ch + 1);
    // A wave whose 32 rows all lie past nq (the last row tile of a head)
    // stages chunks and meets the barriers, but computes and stores nothing.
    if (row0 < a.nq) {
      f32x16 acc[2];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;
      bf16x8 pb[2][3];
      auto read_b = [&](int s, int t, bf16x8 (&dst)[3]) {
        const int off = (32 * t + c) * RS + 32 * s + 16 * g;
#pragma unroll
        for (int q = 0; q < 3; ++q) dst[q] = *reinterpret_cast<const bf16x8*>(&kp[q][off]);
      };
      if (!bad) {
#pragma unroll
        for (int s = 0; s < KST; ++s) {
          read_b(s, 0, pb[0]);
          read_b(s, 1, pb[1]);
          tile_step2(pa[s], pb[0], pb[1], acc[0], acc[1]);
        }
      } else {
#pragma unroll
        for (int s = 0; s < KST; ++s) {
          read_b(s, 0, pb[0]);
          read_b(s, 1, pb[1]);
          tile_step_nf(pa[s], pb[0], acc[0]);
          tile_step_nf(pa[s], pb[1], acc[1]);
        }
      }
      // Scores: rows row0 + 8 (i / 4) + 4 g + i % 4, columns ch * 64 + 32 t + c.
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int col = ch * KC + 32 * t + c;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int row = row0 + 8 * (i / 4) + 4 * g + i % 4;
          const int trow = row - rt * 128;  // row within the tile's resource
          const uint32_t off = (row < a.nq && col < a.nk) ? (uint32_t)(trow * a.nk + col) * 4u : kDrop;
          // Through a scalar: a vector element subscript passed straight to
          // __builtin_bit_cast is read as element 0 by this compiler.
          const float v = acc[t][i];
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), srs, off, 0, 0);
        }
      }
    }
  }
}

template <int D>
hipError_t launch_scores_mfma(RouteArgs a, int BH, hipStream_t stream) {
  a.tiles_per_bh = (a.nq + 127) / 128;
  const int nchunks = (a.nk + 63) / 64;
  const int base = BH * a.tiles_per_bh;
  int splits = (512 + base - 1) / base;  // about two workgroups per CU: one round
  a.col_splits = splits < nchunks ? splits : nchunks;
  hipLaunchKernelGGL((scores_kernel<D>), dim3(base * a.col_splits), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int NPER, int MODE>
hipError_t launch_route_n(RouteArgs a, int BH, hipStream_t stream) {
  // Score rows per wave: the top-k alone runs one row per wave (more rows in
  // flight hide its serial search; two rows per wave measured slower at
  // 14,400 rows and only 2-8 % faster at 28,800-57,600); with the score
  // GEMM, up to 4 rows share each staged key chunk.
  constexpr int RW = (MODE == kTopkOnly || NPER > 32) ? 1 : (NPER <= 16 ? 4 : 2);
  a.tiles_per_bh = (a.nq + 4 * RW - 1) / (4 * RW);
  hipLaunchKernelGGL((route_kernel<NPER, RW, MODE>), dim3(BH * a.tiles_per_bh), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}

template <int NPER, int D>
hipError_t launch_select_mfma_n(RouteArgs a, int BH, hipStream_t stream) {
  a.tiles_per_bh = (a.nq + 15) / 16;
  hipLaunchKernelGGL((select_mfma_kernel<NPER, D>), dim3(BH * a.tiles_per_bh), dim3(256), 0,
                     stream, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_select_mfma(RouteArgs a, int BH, hipStream_t stream) {
  const int per = (a.nk + 63) / 64;
  if (per <= 1) return launch_select_mfma_n<1, D>(a, BH, stream);
  if (per <= 2) return launch_select_mfma_n<2, D>(a, BH, stream);
  if (per <= 4) return launch_select_mfma_n<4, D>(a, BH, stream);
  if (per <= 8) return launch_select_mfma_n<8, D>(a, BH, stream);
  if (per <= 16) return launch_select_mfma_n<16, D>(a, BH, stream);
  return launch_select_mfma_n<32, D>(a, BH, stream);
}

template <int MODE>
hipError_t launch_route(RouteArgs a, int BH, hipStream_t stream) {
  const int per = (a.nk + 63) / 64;
  if (MODE == kScoresOnly) {
    if (a.D == 128) return launch_scores_mfma<128>(a, BH, stream);
    if (a.D == 64) return launch_scores_mfma<64>(a, BH, stream);
  }
  // Fused routing on fp32 MFMA for the common head dims (score rows up to
  // 2048 columns fit the LDS row buffer); the vector-ALU kernel covers the
  // rest.
  if (MODE == kSelect && per <= 32) {
    if (a.D == 128) return launch_select_mfma<128>(a, BH, stream);
    if (a.D == 64) return launch_select_mfma<64>(a, BH, stream);
  }
  if (per <= 1) return launch_route_n<1, MODE>(a, BH, stream);
  if (per <= 2) return launch_route_n<2, MODE>(a, BH, stream);
  if (per <= 4) return launch_route_n<4, MODE>(a, BH, stream);
  if (per <= 8) return launch_route_n<8, MODE>(a, BH, stream);
  if (per <= 16) return launch_route_n<16, MODE>(a, BH, stream);
  if (per <= 32) return launch_route_n<32, MODE>(a, BH, stream);
  return launch_route_n<64, MODE>(a, BH, stream);
}

}  // namespace

bool select_supported(int nk, int D) {
  return nk >= 1 && nk <= kMaxPer * 64 && D >= 4 && D <= kMaxD && D % 4 == 0;
}

hipError_t launch_scores(const float* qbar, const float* kbar, int B, int H, int nq, int nk,
                         int D, float* score, hipStream_t stream) {
  RouteArgs a{};
  a.qbar = qbar;
  a.kbar = kbar;
  a.score_out = score;
  a.H = H;
  a.nq = nq;
  a.nk = nk;
  a.D = D;
  return launch_route<kScoresOnly>(a, B * H, stream);
}

hipError_t launch_topk(const float* score, int B, int H, int nq, int nk, int top_k,
                       int32_t* idx, hipStream_t stream) {
  RouteArgs a{};
  a.score_in = score;
  a.idx = idx;
  a.H = H;
  a.nq = nq;
  a.nk = nk;
  a.top_k = top_k;
  return launch_route<kTopkOnly>(a, B * H, stream);
}

hipError_t launch_select(const float* qbar, const float* kbar, int B, int H, int nq, int nk,
                         int D, int top_k, int32_t* idx, hipStream_t stream) {
  RouteArgs a{};
  a.qbar = qbar;
  a.kbar = kbar;
  a.idx = idx;
  a.H = H;
  a.nq = nq;
  a.nk = nk;
  a.D = D;
  a.top_k = top_k;
  return launch_route<kSelect>(a, B * H, stream);
}

}  // namespace lcv
