// Sparse attention over selected 64-token KV blocks (block sparse attention
// forward), for gfx950.
//
// Semantics follow bsa_attention (longcat_video/models/block_sparse_attention.py:201-250):
// every query row of q-block n attends, with softmax(sm_scale * q.k), to all
// keys of the KV blocks listed for n, and to nothing else.  The reference gets
// there with a dense [B,H,S,S] mask (-1e9 where not routed) and dense SDPA;
// masked entries contribute exactly zero, so walking only the listed blocks
// with an online softmax (as the reference's own kernels do,
// longcat_video/models/block_sparse_attention_metal.py:75-164, 572-712, 829-962)
// gives the same result.
//
// MFMA kernel (fp16 / bf16, D in {64, 128}):
//   * one workgroup (2 waves) per (b, h, q-block); wave w owns query rows
//     32w..32w+31 of the block;
//   * the wave's Q tile stays in registers as the B operand of
//     S^T = K Q^T (v_mfma_f32_32x32x16_{f16,bf16}, fp32 accumulate);
//   * S^T's accumulator layout (lane = query column, 16 keys per tile) is
//     exactly the B-operand layout of O^T = V^T P^T once the key order inside
//     each 16-key step is relabelled, so P never leaves registers and every
//     lane owns one query row: the online-softmax max/sum need a single
//     cross-lane exchange (lane ^ 32) and the O rescale is lane-local;
//   * K is staged in LDS row-major (row stride D+8 halves), V transposed
//     (V^T, row stride 64+8 halves) with key bits 2 and 3 swapped, which puts
//     the 8 keys a lane feeds to one MFMA step at adjacent addresses -- every
//     LDS operand read is one conflict-free 16-byte ds_read;
//   * the next selected block is fetched into registers while the current one
//     is multiplied (register double buffering), and workgroups are ordered
//     so each XCD sweeps the q-blocks of one head (shared K/V in its L2).
//
// Vector-ALU kernel (any dtype, D in {16, 32, 64, 128, 256}): 64 rows x 4
// lanes per workgroup, fp32 throughout; used for fp32 inputs and head dims
// without an MFMA tiling.
#include "bsa_common.h"

namespace lcv {
namespace {

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int next_valid(const int32_t* list, int j, int top_k, int nb) {
  while (j < top_k) {
    const int n = uniform_i32(list[j]);
    if (n >= 0 && n < nb) break;
    ++j;
  }
  return j;
}

// Position of key `key` (0..63) inside a 16-key MFMA step of the V^T tile:
// swap bits 2 and 3.
__device__ __forceinline__ int vt_pos(int key) {
  return (key & ~0xC) | ((key & 0x4) << 1) | ((key & 0x8) >> 1);
}

template <typename T>
struct Mfma;

template <>
struct Mfma<f16> {
  typedef f16x8 vec8;
  __device__ static f32x16 mma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<bf16> {
  typedef bf16x8 vec8;
  __device__ static f32x16 mma(vec8 a, vec8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <typename T, int D>
struct MfmaCfg {
  static constexpr int kThreads = 128;
  static constexpr int KS = D + 8;         // K tile row stride (elements)
  static constexpr int VS = 64 + 8;        // V^T tile row stride (elements)
  static constexpr int DC = D / 8;         // 16-byte chunks per row
  static constexpr int kPieces = 64 * DC / kThreads;  // K 16-byte loads / thread
  static constexpr int vItems = 16 * DC / kThreads;   // V (4 keys x 8 d) items / thread
  static_assert(kPieces >= 1 && vItems >= 1, "tile too small for the workgroup");
};

template <typename T, int D>
__global__ __launch_bounds__(128) void attn_mfma_kernel(AttnParams p) {
  typedef MfmaCfg<T, D> C;
  typedef typename Mfma<T>::vec8 vec8;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[64 * C::KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * C::VS];

  const int wid = xcd_linear_work_id(blockIdx.x, gridDim.x);
  const int bh = wid / p.nb;
  const int qb = wid - bh * p.nb;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int tid = threadIdx.x;
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int l32 = lane % 32;
  const int g = lane / 32;

  const T* qbase = reinterpret_cast<const T*>(p.q) + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const T* kbase = reinterpret_cast<const T*>(p.k) + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  T* obase = reinterpret_cast<T*>(p.out) + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;

  // ---- Q tile: B operand of S^T = K Q^T; lane holds Q[row][16ks + 8g .. +8].
  const int32_t qtok = block_base_token(p.g, qb) + voxel_row_offset(p.g, 32 * wave + l32);
  vec8 qf[D / 16];
  {
    const T* qrow = qbase + (int64_t)qtok * p.q_ss + 8 * g;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks)
      qf[ks] = __builtin_bit_cast(vec8, *reinterpret_cast<const u32x4*>(qrow + 16 * ks));
  }

  // ---- Fixed per-thread staging coordinates.
  int32_t koff[C::kPieces];
  int kcol[C::kPieces];
  int klds[C::kPieces];
#pragma unroll
  for (int it = 0; it < C::kPieces; ++it) {
    const int pidx = tid + C::kThreads * it;
    const int row = pidx / C::DC;
    const int c = pidx % C::DC;
    koff[it] = voxel_row_offset(p.g, row);
    kcol[it] = 8 * c;
    klds[it] = row * C::KS + 8 * c;
  }
  int32_t voff[C::vItems][4];
  int vcol[C::vItems];
  int vlds[C::vItems];
#pragma unroll
  for (int it = 0; it < C::vItems; ++it) {
    const int pidx = tid + C::kThreads * it;
    const int a4 = pidx % 16;  // key quad
    const int c = pidx / 16;   // d chunk
#pragma unroll
    for (int r = 0; r < 4; ++r) voff[it][r] = voxel_row_offset(p.g, 4 * a4 + r);
    vcol[it] = 8 * c;
    vlds[it] = (8 * c) * C::VS + vt_pos(4 * a4);
  }

  u32x4 kreg[C::kPieces];
  u32x4 vreg[C::vItems][4];
  auto load_tile = [&](int n) {
    const int32_t tok0 = block_base_token(p.g, n);
#pragma unroll
    for (int it = 0; it < C::kPieces; ++it)
      kreg[it] = *reinterpret_cast<const u32x4*>(kbase + (int64_t)(tok0 + koff[it]) * p.k_ss + kcol[it]);
#pragma unroll
    for (int it = 0; it < C::vItems; ++it)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        vreg[it][r] =
            *reinterpret_cast<const u32x4*>(vbase + (int64_t)(tok0 + voff[it][r]) * p.v_ss + vcol[it]);
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int it = 0; it < C::kPieces; ++it) *reinterpret_cast<u32x4*>(&Ks[klds[it]]) = kreg[it];
#pragma unroll
    for (int it = 0; it < C::vItems; ++it) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {  // 32-bit word m = elements 2m, 2m+1 of each row
        const uint32_t w0 = vreg[it][0][m], w1 = vreg[it][1][m];
        const uint32_t w2 = vreg[it][2][m], w3 = vreg[it][3][m];
        u32x2 lo, hi;
        lo[0] = (w0 & 0xffffu) | (w1 << 16);
        lo[1] = (w2 & 0xffffu) | (w3 << 16);
        hi[0] = (w0 >> 16) | (w1 & 0xffff0000u);
        hi[1] = (w2 >> 16) | (w3 & 0xffff0000u);
        *reinterpret_cast<u32x2*>(&Vt[vlds[it] + (2 * m) * C::VS]) = lo;
        *reinterpret_cast<u32x2*>(&Vt[vlds[it] + (2 * m + 1) * C::VS]) = hi;
      }
    }
  };

  f32x16 oacc[D / 32];
#pragma unroll
  for (int md = 0; md < D / 32; ++md)
#pragma unroll
    for (int i = 0; i < 16; ++i) oacc[md][i] = 0.0f;
  float m_run = -__builtin_inff();
  float l_run = 0.0f;
  const float sl2 = p.scale_log2;

  const int32_t* list = p.idx + ((int64_t)bh * p.nb + qb) * p.top_k;
  int j = next_valid(list, 0, p.top_k, p.nb);
  if (j < p.top_k) load_tile(uniform_i32(list[j]));

  while (j < p.top_k) {
    __syncthreads();  // every wave is done with the previous tile
    store_tile();
    __syncthreads();  // tile visible
    const int jn = next_valid(list, j + 1, p.top_k, p.nb);
    if (jn < p.top_k) load_tile(uniform_i32(list[jn]));  // in flight during the math

    // S^T (64 keys x 32 queries) = K Q^T.
    f32x16 sacc[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) sacc[mt][i] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const vec8 kf = __builtin_bit_cast(
            vec8, *reinterpret_cast<const u32x4*>(&Ks[(32 * mt + l32) * C::KS + 16 * ks + 8 * g]));
        sacc[mt] = Mfma<T>::mma(kf, qf[ks], sacc[mt]);
      }
    }

    // Online softmax for this lane's query row (keys split between g = 0, 1).
    float t[32];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) t[16 * mt + i] = sacc[mt][i] * sl2;
    float mx = t[0];
#pragma unroll
    for (int i = 1; i < 32; ++i) mx = fmaxf(mx, t[i]);
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float corr = fast_exp2(m_run - m_new);
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      t[i] = fast_exp2(t[i] - m_new);
      psum += t[i];
    }
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int md = 0; md < D / 32; ++md)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[md][i] *= corr;

    // P^T as the B operand: step s takes accumulator values 8s .. 8s+7.
    vec8 pf[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) pf[s][jj] = from_f32<T>(t[8 * s + jj]);

    // O^T (D x 32 queries) += V^T P^T.
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int md = 0; md < D / 32; ++md) {
        const vec8 vf = __builtin_bit_cast(
            vec8, *reinterpret_cast<const u32x4*>(&Vt[(32 * md + l32) * C::VS + 16 * s + 8 * g]));
        oacc[md] = Mfma<T>::mma(vf, pf[s], oacc[md]);
      }
    }
    j = jn;
  }

  // ---- Normalise and store: lane owns O[row][32md + 8(i/4) + 4g + (i%4)].
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
  T* orow = obase + (int64_t)qtok * p.o_ss;
#pragma unroll
  for (int md = 0; md < D / 32; ++md) {
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      u32x2 w;
      w[0] = bits16(from_f32<T>(oacc[md][4 * i4 + 0] * inv)) |
             (bits16(from_f32<T>(oacc[md][4 * i4 + 1] * inv)) << 16);
      w[1] = bits16(from_f32<T>(oacc[md][4 * i4 + 2] * inv)) |
             (bits16(from_f32<T>(oacc[md][4 * i4 + 3] * inv)) << 16);
      *reinterpret_cast<u32x2*>(orow + 32 * md + 8 * i4 + 4 * g) = w;
    }
  }
}

// ---------------------------------------------------------------------------
// Vector-ALU kernel: workgroup = 64 query rows x 4 lanes; lane (r, quarter)
// owns D/4 columns of q and o.  K/V are staged 32 keys at a time as fp32.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_valu_kernel(AttnParams p) {
  constexpr int DQ = D / 4;
  constexpr int KH = D >= 256 ? 16 : 32;  // keys staged per pass (LDS <= 32 KB)
  __shared__ float Kf[KH * D];
  __shared__ float Vf[KH * D];

  const int wid = xcd_linear_work_id(blockIdx.x, gridDim.x);
  const int bh = wid / p.nb;
  const int qb = wid - bh * p.nb;
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int tid = threadIdx.x;
  const int r = tid / 4;
  const int qd = tid % 4;

  const T* qbase = reinterpret_cast<const T*>(p.q) + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const T* kbase = reinterpret_cast<const T*>(p.k) + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  T* obase = reinterpret_cast<T*>(p.out) + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;

  const int32_t qtok = block_base_token(p.g, qb) + voxel_row_offset(p.g, r);
  float qv[DQ], ov[DQ];
#pragma unroll
  for (int dd = 0; dd < DQ; ++dd) {
    qv[dd] = to_f32(qbase[(int64_t)qtok * p.q_ss + qd * DQ + dd]);
    ov[dd] = 0.0f;
  }
  float m_run = -__builtin_inff();
  float l_run = 0.0f;
  const float sl2 = p.scale_log2;
  const int32_t* list = p.idx + ((int64_t)bh * p.nb + qb) * p.top_k;

  for (int j = next_valid(list, 0, p.top_k, p.nb); j < p.top_k;
       j = next_valid(list, j + 1, p.top_k, p.nb)) {
    const int32_t tok0 = block_base_token(p.g, uniform_i32(list[j]));
    for (int half = 0; half < 64; half += KH) {
      __syncthreads();
      for (int i = tid; i < KH * D; i += 256) {
        const int kr = i / D;
        const int d = i - kr * D;
        const int32_t tok = tok0 + voxel_row_offset(p.g, half + kr);
        Kf[i] = to_f32(kbase[(int64_t)tok * p.k_ss + d]);
        Vf[i] = to_f32(vbase[(int64_t)tok * p.v_ss + d]);
      }
      __syncthreads();
      float s[KH];
#pragma unroll
      for (int kk = 0; kk < KH; ++kk) {
        float part = 0.0f;
#pragma unroll
        for (int dd = 0; dd < DQ; ++dd) part = fmaf(qv[dd], Kf[kk * D + qd * DQ + dd], part);
        part += __shfl_xor(part, 1);
        part += __shfl_xor(part, 2);
        s[kk] = part * sl2;
      }
      float mx = s[0];
#pragma unroll
      for (int kk = 1; kk < KH; ++kk) mx = fmaxf(mx, s[kk]);
      const float m_new = fmaxf(m_run, mx);
      const float corr = fast_exp2(m_run - m_new);
      l_run *= corr;
#pragma unroll
      for (int dd = 0; dd < DQ; ++dd) ov[dd] *= corr;
#pragma unroll
      for (int kk = 0; kk < KH; ++kk) {
        const float pe = fast_exp2(s[kk] - m_new);
        l_run += pe;
#pragma unroll
        for (int dd = 0; dd < DQ; ++dd) ov[dd] = fmaf(pe, Vf[kk * D + qd * DQ + dd], ov[dd]);
      }
      m_run = m_new;
    }
  }
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
#pragma unroll
  for (int dd = 0; dd < DQ; ++dd)
    obase[(int64_t)qtok * p.o_ss + qd * DQ + dd] = from_f32<T>(ov[dd] * inv);
}

template <typename T, int D>
hipError_t launch_mfma(const AttnParams& p, hipStream_t stream) {
  const int grid = p.B * p.H * p.nb;
  hipLaunchKernelGGL((attn_mfma_kernel<T, D>), dim3(grid), dim3(128), 0, stream, p);
  return hipGetLastError();
}

template <typename T, int D>
hipError_t launch_valu(const AttnParams& p, hipStream_t stream) {
  const int grid = p.B * p.H * p.nb;
  hipLaunchKernelGGL((attn_valu_kernel<T, D>), dim3(grid), dim3(256), 0, stream, p);
  return hipGetLastError();
}

template <typename T>
hipError_t launch_valu_d(const AttnParams& p, int D, hipStream_t stream) {
  switch (D) {
    case 16: return launch_valu<T, 16>(p, stream);
    case 32: return launch_valu<T, 32>(p, stream);
    case 64: return launch_valu<T, 64>(p, stream);
    case 128: return launch_valu<T, 128>(p, stream);
    case 256: return launch_valu<T, 256>(p, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool attn_uses_mfma(int dtype, int D) {
  return (dtype == LCV_BSA_F16 || dtype == LCV_BSA_BF16) && (D == 64 || D == 128);
}

bool attn_supported(int dtype, int D) {
  return D == 16 || D == 32 || D == 64 || D == 128 || D == 256;
}

hipError_t launch_attn(const AttnParams& p, int dtype, int D, hipStream_t stream) {
  if (attn_uses_mfma(dtype, D)) {
    if (dtype == LCV_BSA_F16)
      return D == 64 ? launch_mfma<f16, 64>(p, stream) : launch_mfma<f16, 128>(p, stream);
    return D == 64 ? launch_mfma<bf16, 64>(p, stream) : launch_mfma<bf16, 128>(p, stream);
  }
  switch (dtype) {
    case LCV_BSA_F16: return launch_valu_d<f16>(p, D, stream);
    case LCV_BSA_BF16: return launch_valu_d<bf16>(p, D, stream);
    default: return launch_valu_d<float>(p, D, stream);
  }
}

}  // namespace lcv
