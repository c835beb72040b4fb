// Block routing: fp32 block scores qbar . kbar^T and per-row top-k.
//
// The score GEMM runs on fp32 MFMA for head dims 64 and 128 (nk <= 2048) and
// on fp32 FMAs otherwise; either way each score is an fp32 dot product, and
// selection is exact given score margins well above fp32 rounding.
//
// Follows block_routing_scores + topk_block_indices
// (longcat_video/models/block_sparse_attention.py:107-134).  The reference
// materialises the [B,H,nq,nk] score tensor and runs argpartition; here a
// wave computes whole score rows straight into registers in the layout its
// top-k needs (lane l holds columns l, l+64, l+128, ...), so the fused path
// never writes scores to memory.
//
// Top-k is an exact radix select on order-preserving 32-bit keys: a 32-step
// binary search finds the k-th largest key with ballot/popcount counts (over
// the keys above a cheap exact lower bound, compacted, when k <= 128), then
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

// Largest t with #(key >= t) >= k, built bit by bit over R keys per lane
// (padding keys are 0 and never reach a candidate >= 1).  Once a candidate
// at or above `floor` has exactly k keys at or above it, those keys are the
// top k and the remaining bits cannot change the selection.
template <int R>
__device__ uint32_t kth_key(const uint32_t (&key)[R], int k, uint32_t floor) {
  uint32_t thr = 0u;
  for (int bit = 31; bit >= 0; --bit) {
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

template <int R>
__device__ uint32_t kth_key_compacted(const uint32_t* buf, int total, int k, uint32_t floor) {
  const int lane = lane_id();
  uint32_t key[R];
#pragma unroll
  for (int r = 0; r < R; ++r) key[r] = lane + 64 * r < total ? buf[lane + 64 * r] : 0u;
  return kth_key<R>(key, k, floor);
}

// Exact top-k of one score row held as sc[e] = score[e*64 + lane], e < NPER.
// Writes the k selected column indices, ascending, to out[0..k).  buf:
// kCompactCap words of this wave's LDS.
//
// For k <= 64 (and nk >= 64) a lower bound on the k-th largest key comes
// first: every lane's largest key is >= L = their minimum, so at least
// 64 >= k keys are >= L and the k-th largest key is among the keys >= L.
// Those (typically a quarter of the row) are compacted into 4 or 8
// registers per lane and searched there; counts at candidates >= L equal
// the full row's, below L both are >= k, so the threshold is the full row's.
template <int NPER>
__device__ void wave_topk(const float (&sc)[NPER], int nk, int k, int32_t* out, uint32_t* buf) {
  const int lane = lane_id();
  uint32_t key[NPER];
#pragma unroll
  for (int e = 0; e < NPER; ++e) {
    const int col = e * 64 + lane;
    key[e] = col < nk ? order_key(sc[e]) : 0u;
  }
  uint32_t thr = 0u;
  bool found = false;
  if (k <= 64 && nk >= 64) {  // wave-uniform
    uint32_t lane_max = 0u;
#pragma unroll
    for (int e = 0; e < NPER; ++e) lane_max = key[e] > lane_max ? key[e] : lane_max;
    const uint32_t L = wave_min_u32(lane_max);
    int total = 0;
#pragma unroll
    for (int e = 0; e < NPER; ++e) {
      const bool in = e * 64 + lane < nk && key[e] >= L;
      const uint64_t msk = ballot64(in);
      const int pos = total + (int)mbcnt64(msk);
      if (in && pos < kCompactCap) buf[pos] = key[e];
      total += __popcll(msk);
    }
    if (total <= 256) {
      thr = kth_key_compacted<4>(buf, total, k, L);
      found = true;
    } else if (total <= kCompactCap) {
      thr = kth_key_compacted<8>(buf, total, k, L);
      found = true;
    }
  }
  if (!found) thr = kth_key<NPER>(key, k, 0u);

  int gt = 0;
#pragma unroll
  for (int e = 0; e < NPER; ++e) gt += __popcll(ballot64(key[e] > thr));
  const int need_eq = k - gt;
  int run_sel = 0, run_eq = 0;
#pragma unroll
  for (int e = 0; e < NPER; ++e) {
    const int col = e * 64 + lane;
    const bool valid = col < nk;
    const bool is_gt = valid && key[e] > thr;
    const bool is_eq = valid && key[e] == thr;
    const uint64_t eqm = ballot64(is_eq);
    const int eq_rank = run_eq + (int)mbcnt64(eqm);
    const bool sel = is_gt || (is_eq && eq_rank < need_eq);
    const uint64_t selm = ballot64(sel);
    if (sel) out[run_sel + (int)mbcnt64(selm)] = col;
    run_sel += __popcll(selm);
    run_eq += __popcll(eqm);
  }
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
  __shared__ uint32_t tk_buf[4][kCompactCap];
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

// Score rows on fp32 MFMA (v_mfma_f32_16x16x4_f32).  One workgroup = 16
// q-block rows of one (b, h); wave w computes the 16-column score tiles
// w, w + 4, ... .  Operands come straight from global memory into registers:
// k-step s = 4 s4 + u of lane (c, kg) (c = lane % 16, kg = lane / 16) pairs
// dim 16 s4 + 4 kg + u of q-block row c (A) and of key row 16t + c (B), so
// the four kg lanes of a row load 64 contiguous bytes per instruction (16
// cache lines per wave load, not 64).  The accumulator holds
// S[4kg + i][16t + c].  The 16 x nk score rows are gathered in LDS and each
// wave runs wave_topk on four of them: routing without a score buffer.
template <int NPER, int D>
__global__ __launch_bounds__(256) void select_mfma_kernel(RouteArgs a) {
  constexpr int QR = 16;
  constexpr int DQ = D / 4;                 // dims per lane group
  constexpr int LDSW = NPER * 64 + 4;       // score row stride (floats)
  __shared__ __attribute__((aligned(16))) float srow[QR * LDSW];
  __shared__ uint32_t tk_buf[4][kCompactCap];
  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int c = lane % 16;
  const int kg = lane / 16;
  const int bh = blockIdx.x / a.tiles_per_bh;
  const int row0 = (blockIdx.x - bh * a.tiles_per_bh) * QR;
  const float* qb = a.qbar + (int64_t)bh * a.nq * D;
  const float* kb = a.kbar + (int64_t)bh * a.nk * D;

  float qa[DQ];
  {
    const int row = row0 + c;
#pragma unroll
    for (int s4 = 0; s4 < DQ / 4; ++s4) {
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (row < a.nq) v = *reinterpret_cast<const f32x4*>(qb + (int64_t)row * D + 16 * s4 + 4 * kg);
#pragma unroll
      for (int u = 0; u < 4; ++u) qa[4 * s4 + u] = v[u];
    }
  }
  const int ntiles = (a.nk + 15) / 16;
  auto load_b = [&](int t, float (&kv)[DQ]) {
    const int key = 16 * t + c;
#pragma unroll
    for (int s4 = 0; s4 < DQ / 4; ++s4) {
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (key < a.nk) v = *reinterpret_cast<const f32x4*>(kb + (int64_t)key * D + 16 * s4 + 4 * kg);
#pragma unroll
      for (int u = 0; u < 4; ++u) kv[4 * s4 + u] = v[u];
    }
  };
  float kv0[DQ], kv1[DQ];
  int t = wave;
  if (t < ntiles) load_b(t, kv0);
  auto tile = [&](int tt, const float (&kv)[DQ]) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < DQ; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[s], kv[s], acc, 0, 0, 0);
    const int col = 16 * tt + c;
#pragma unroll
    for (int i = 0; i < 4; ++i) srow[(4 * kg + i) * LDSW + col] = acc[i];
  };
  for (; t < ntiles; t += 8) {
    if (t + 4 < ntiles) load_b(t + 4, kv1);
    tile(t, kv0);
    if (t + 4 >= ntiles) break;
    if (t + 8 < ntiles) load_b(t + 8, kv0);
    tile(t + 4, kv1);
  }
  __syncthreads();
#pragma unroll 1
  for (int r = wave; r < QR; r += 4) {
    const int row = row0 + r;
    if (row >= a.nq) break;  // wave-uniform; rows only grow
    float sc[NPER];
#pragma unroll
    for (int e = 0; e < NPER; ++e) sc[e] = srow[r * LDSW + e * 64 + lane];
    wave_topk<NPER>(sc, a.nk, a.top_k, a.idx + ((int64_t)bh * a.nq + row) * a.top_k,
                    tk_buf[wave]);
  }
}

// Score matrix S = qbar kbar^T on fp32 MFMA (v_mfma_f32_16x16x4_f32), written
// to memory.  One workgroup = 4 waves x 16 q-block rows (64 rows) of one
// (b, h) over a range of 64-key chunks (col_splits ranges per row tile, so
// that small heads still fill the GPU).  A chunk's kbar rows are staged in
// LDS (row stride D + 4 floats: the 16-byte operand reads are conflict free)
// from coalesced 16-byte loads, which for the next chunk are in flight while
// the current chunk's MFMAs run.  Each wave keeps its rows' qbar in
// registers and runs the chunk's four 16-key tiles as four interleaved MFMA
// chains.  k-step s = 4 s4 + u of lane (c, kg) pairs dim 16 s4 + 4 kg + u of
// q-block row c and of key row 16t + c; the accumulator holds
// S[4kg + i][16t + c].
template <int D>
__global__ __launch_bounds__(256) void scores_kernel(RouteArgs a) {
  constexpr int KC = 64;              // keys per chunk
  constexpr int KS = D + 4;           // LDS row stride (floats)
  constexpr int DQ = D / 4;           // k-steps per tile
  constexpr int D4 = D / 4;           // 16-byte pieces per row
  constexpr int kLoads = KC * D4 / 256;
  static_assert(kLoads * 256 == KC * D4, "chunk loads split evenly over the workgroup");
  __shared__ __attribute__((aligned(16))) float kch[KC * KS];
  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int c = lane % 16;
  const int kg = lane / 16;
  const int per_bh = a.tiles_per_bh * a.col_splits;
  const int bh = blockIdx.x / per_bh;
  const int rem = blockIdx.x - bh * per_bh;
  const int rt = rem / a.col_splits;
  const int cs = rem - rt * a.col_splits;
  const int row0 = rt * 64 + wave * 16;
  const int nchunks = (a.nk + KC - 1) / KC;
  const int ch0 = (int)((int64_t)cs * nchunks / a.col_splits);
  const int ch1 = (int)((int64_t)(cs + 1) * nchunks / a.col_splits);
  const float* qb = a.qbar + (int64_t)bh * a.nq * D;
  const float* kb = a.kbar + (int64_t)bh * a.nk * D;
  float* so = a.score_out + (int64_t)bh * a.nq * a.nk;

  float qa[DQ];
  {
    const int row = row0 + c;
#pragma unroll
    for (int s4 = 0; s4 < DQ / 4; ++s4) {
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (row < a.nq) v = *reinterpret_cast<const f32x4*>(qb + (int64_t)row * D + 16 * s4 + 4 * kg);
#pragma unroll
      for (int u = 0; u < 4; ++u) qa[4 * s4 + u] = v[u];
    }
  }
  f32x4 st[kLoads];
  auto load_chunk = [&](int ch) {
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int i = tid + 256 * u;
      const int key = ch * KC + i / D4;
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      if (key < a.nk) v = *reinterpret_cast<const f32x4*>(kb + (int64_t)key * D + 4 * (i % D4));
      st[u] = v;
    }
  };
  if (ch0 < ch1) load_chunk(ch0);
  for (int ch = ch0; ch < ch1; ++ch) {
    __syncthreads();  // the previous chunk is consumed
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
      const int i = tid + 256 * u;
      *reinterpret_cast<f32x4*>(kch + (i / D4) * KS + 4 * (i % D4)) = st[u];
    }
    __syncthreads();
    if (ch + 1 < ch1) load_chunk(ch + 1);
    f32x4 acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // The key operands of step s4 + 1 are read while the MFMAs of step s4
    // run (scheduling groups keep the compiler from sinking the reads).
    f32x4 kv[2][4];
    auto read_kv = [&](int s4, f32x4* dst) {
#pragma unroll
      for (int t = 0; t < 4; ++t)
        dst[t] = *reinterpret_cast<const f32x4*>(kch + (16 * t + c) * KS + 16 * s4 + 4 * kg);
    };
    read_kv(0, kv[0]);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);  // DS reads
#pragma unroll
    for (int s4 = 0; s4 < DQ / 4; ++s4) {
      if (s4 + 1 < DQ / 4) read_kv(s4 + 1, kv[(s4 + 1) & 1]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[4 * s4 + u], kv[s4 & 1][t][u], acc[t], 0,
                                                        0, 0);
        if (s4 + 1 < DQ / 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);  // MFMA
      }
    }
    // Scores: rows row0 + 4kg + i, columns ch*64 + 16t + c.  Interior tiles
    // store without per-element checks.
    float* srow = so + (int64_t)(row0 + 4 * kg) * a.nk + ch * KC + c;
    if (row0 + 16 <= a.nq && (ch + 1) * KC <= a.nk) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) srow[(int64_t)i * a.nk + 16 * t] = acc[t][i];
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int col = ch * KC + 16 * t + c;
        if (col < a.nk) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int row = row0 + 4 * kg + i;
            if (row < a.nq) so[(int64_t)row * a.nk + col] = acc[t][i];
          }
        }
      }
    }
  }
}

template <int D>
hipError_t launch_scores_mfma(RouteArgs a, int BH, hipStream_t stream) {
  a.tiles_per_bh = (a.nq + 63) / 64;
  const int nchunks = (a.nk + 63) / 64;
  const int base = BH * a.tiles_per_bh;
  int splits = (1024 + base - 1) / base;  // about four workgroups per CU
  a.col_splits = splits < nchunks ? splits : nchunks;
  hipLaunchKernelGGL((scores_kernel<D>), dim3(base * a.col_splits), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int NPER, int MODE>
hipError_t launch_route_n(RouteArgs a, int BH, hipStream_t stream) {
  // Score rows per wave: the top-k alone runs one row per wave (more rows in
  // flight hide its serial search); with the score GEMM, up to 4 rows share
  // each staged key chunk.
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
