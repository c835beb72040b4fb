// Pre-BSA preparation of q and k in one pass: per-head RMSNorm (fp32 math),
// 3D RoPE, and the block means the routing needs.
//
// Follows the attention layer ahead of BSA (longcat_video/models/attention.py:
// 191-201):
//   q = RMSNorm_FP32(q)  -- blocks.py:55-72: x_f32 * rsqrt(mean(x_f32^2) + eps),
//                           rounded to the input dtype, times the weight in
//                           that dtype;
//   q = rope_3d(q)       -- rope_3d.py:107-128: widened to fp32,
//                           x*cos + rotate_half(x)*sin, rounded back;
// (the same for k), followed by mean_pool_blocks_3d of the result
// (block_sparse_attention.py:67-104).  The reference runs these as separate
// full-tensor passes; here one wave reads each row of a block once, writes
// the prepared row and accumulates the block mean of the written values.
//
// RoPE angles come from a per-axis table built by the caller (cos and sin of
// position * inverse frequency for the t, h and w parts of the head dim),
// staged in LDS once per (persistent) workgroup.  The RoPE grid is the latent grid; the
// BSA blocks may be a different view of the same tokens (e.g. contiguous
// 64-token blocks), so the two geometries are separate arguments.
#include <algorithm>

#include "norm_common.h"

namespace lcv {
namespace {

constexpr int kPrepWaves = 4;

struct PrepArgs {
  Tensor4 in[2];
  Tensor4 out[2];
  const void* weight[2];  // [D] in the tensor dtype, or null (weight 1)
  float* mean[2];         // [B, H, nb, D] fp32
  const float* table;     // cos_t, sin_t, cos_h, sin_h, cos_w, sin_w
  int32_t H, D, nb;
  int32_t rT, rH, rW;     // RoPE grid
  int32_t dt, dh;         // RoPE dims of the t and h parts (w takes the rest)
  int32_t table_len;
  int32_t total_items;
  float eps;
  float rcp_plane, rcp_w;  // 1 / (rH * rW), 1 / rW
  float neg_zero, one;     // -0.0f and 1.0f (FMA operands the compiler cannot fold)
  Geom g;
  FastDiv per_block;      // 2 * B * H: items per BSA block index
  FastDiv heads;          // H
};

// Quotient of n by d for n < 2^22 from an fp32 reciprocal: (n + 1/2) / d is
// at least 1/(2d) away from an integer, more than the rounding error of
// (n + 1/2) * fl(1/d) (under 2^-23 relative) can cover for n < 2^22.
__device__ __forceinline__ uint32_t small_div(uint32_t n, float rcp) {
  return (uint32_t)__builtin_fmaf((float)n, rcp, 0.5f * rcp);
}

// The table as staged in LDS: per axis, (cos, sin) interleaved per column, so
// a pair's two factors are one 8-byte read.  Axis a's region starts where its
// cos part starts in the caller's layout (the regions have the same sizes).
__device__ __forceinline__ int lds_slot(const PrepArgs& a, int i) {
  const int ht = a.dt / 2, hh = a.dh / 2, hw = (a.D - a.dt - a.dh) / 2;
  const int nt = a.rT * ht, nh = a.rH * hh, nw = a.rW * hw;
  int base = 0, n = nt;
  if (i >= 2 * nt + 2 * nh) {
    base = 2 * nt + 2 * nh;
    n = nw;
  } else if (i >= 2 * nt) {
    base = 2 * nt;
    n = nh;
  }
  const int j = i - base;
  return j < n ? base + 2 * j : base + 2 * (j - n) + 1;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void prep_kernel(PrepArgs a) {
  constexpr int LPR = D / 8;       // lanes per row (8 elements per lane)
  constexpr int RPS = 64 / LPR;    // rows per step
  extern __shared__ float tab[];  // table_len floats (dynamic)
  __shared__ int64_t row_in[2][64], row_out[2][64];  // element offset of each block row
  __shared__ int32_t row_tok[64];                    // token offset of each block row

  // The workgroup is persistent: the table and the row offsets are staged
  // once and its waves then walk the (block, tensor, b, h) items with a
  // grid-wide stride.
  for (int i = threadIdx.x; i < a.table_len; i += 256) tab[lds_slot(a, i)] = a.table[i];
  if (threadIdx.x < 64) {
    const int32_t t = voxel_row_offset(a.g, threadIdx.x);
    row_tok[threadIdx.x] = t;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      row_in[k][threadIdx.x] = (int64_t)t * a.in[k].ss;
      row_out[k][threadIdx.x] = (int64_t)t * a.out[k].ss;
    }
  }
  __syncthreads();

  const int wave = uniform_i32(threadIdx.x / 64);
  const int lane = threadIdx.x % 64;
  const int c = lane % LPR;  // this lane's 8 dims: 8c .. 8c+7
  // Per pair p (dims 8c + 2p, +1): its axis and its column's offset in that
  // axis' LDS row (in floats).
  const int ht2 = a.dt, hh2 = a.dh, hw2 = D - a.dt - a.dh;  // floats per LDS row
  const int reg_h = a.rT * ht2, reg_w = reg_h + a.rH * hh2;
  int axis[4], col2[4];
#pragma unroll
  for (int pp = 0; pp < 4; ++pp) {
    const int d = 8 * c + 2 * pp;
    axis[pp] = d < a.dt ? 0 : (d < a.dt + a.dh ? 1 : 2);
    col2[pp] = axis[pp] == 0 ? d : (axis[pp] == 1 ? d - a.dt : d - a.dt - a.dh);
  }
  const uint32_t plane = (uint32_t)(a.rH * a.rW);
  const float nz = a.neg_zero, one = a.one;
  const int stride = gridDim.x * kPrepWaves;

  for (int item = blockIdx.x * kPrepWaves + wave; item < a.total_items; item += stride) {
    // Items run head-fastest, so the waves resident together read the q and k
    // heads of the same tokens (adjacent in a fused QKV buffer).
    const uint32_t n = fast_div((uint32_t)item, a.per_block);
    const uint32_t r = (uint32_t)item - n * a.per_block.d;
    const uint32_t bt = fast_div(r, a.heads);
    const int h = (int)(r - bt * a.heads.d);
    const int tensor = (int)(bt & 1u);
    const int b = (int)(bt >> 1);
    const int bh = b * a.H + h;
    const int32_t tok0 = block_base_token(a.g, (int32_t)n);
    const Tensor4 xi = a.in[tensor];
    const Tensor4 xo = a.out[tensor];
    const T* src = reinterpret_cast<const T*>(xi.ptr) + (int64_t)b * xi.sb + (int64_t)h * xi.sh +
                   (int64_t)tok0 * xi.ss + 8 * c;
    T* dst = reinterpret_cast<T*>(const_cast<void*>(xo.ptr)) + (int64_t)b * xo.sb + (int64_t)h * xo.sh +
             (int64_t)tok0 * xo.ss + 8 * c;
    u32x4 wr;
    if (a.weight[tensor]) {
      wr = *reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(a.weight[tensor]) + 8 * c);
    } else {
      const uint32_t one = bits16(from_f32<T>(1.0f));
      wr = u32x4{one | (one << 16), one | (one << 16), one | (one << 16), one | (one << 16)};
    }

    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
#pragma unroll 2
    for (int st = 0; st < 64 / RPS; ++st) {
      const int row = st * RPS + lane / LPR;
      // q / k are streamed once: non-temporal loads and stores.
      const u32x4 raw = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + row_in[tensor][row]));
      float x[8];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        x[2 * m] = to_f32(__builtin_bit_cast(T, (uint16_t)(raw[m] & 0xffffu)));
        x[2 * m + 1] = to_f32(__builtin_bit_cast(T, (uint16_t)(raw[m] >> 16)));
      }
      // RMSNorm: the row's sum of squares over its LPR lanes.
      float ss = 0.0f;
#pragma unroll
      // x*x of a 16-bit value is exact in fp32, so the fused form rounds the
      // sum exactly as square-then-add does.
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(x[e], x[e], ss);
      ss = group_sum<LPR>(ss);
      const float rs = rsqrtf(ss * (1.0f / D) + a.eps);
      float y[8];
      norm_scale<T>(x, rs, wr, nz, y);
      // RoPE at the token's grid position: the LDS row of each axis.
      const uint32_t tok = (uint32_t)(tok0 + row_tok[row]);
      const uint32_t pt = small_div(tok, a.rcp_plane);
      const uint32_t prem = tok - __umul24(pt, plane);
      const uint32_t ph = small_div(prem, a.rcp_w);
      const uint32_t pw = prem - __umul24(ph, (uint32_t)a.rW);
      const int at = (int)__umul24(pt, (uint32_t)ht2);
      const int ah = reg_h + (int)__umul24(ph, (uint32_t)hh2);
      const int aw = reg_w + (int)__umul24(pw, (uint32_t)hw2);
      uint32_t packed[4];
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        const int slot = (axis[pp] == 0 ? at : (axis[pp] == 1 ? ah : aw)) + col2[pp];
        const float2 f = *reinterpret_cast<const float2*>(tab + slot);
        const float cs = f.x, sn = f.y;
        const float u = y[2 * pp], v = y[2 * pp + 1];
        // x*cos + rotate_half(x)*sin, rounded per product and sum.
        const T o0 = round_from_f32<T>(mul1(u, cs, nz) - mul1(v, sn, nz));
        const T o1 = round_from_f32<T>(mul1(v, cs, nz) + mul1(u, sn, nz));
        acc[2 * pp] = __builtin_fmaf(to_f32(o0), one, acc[2 * pp]);
        acc[2 * pp + 1] = __builtin_fmaf(to_f32(o1), one, acc[2 * pp + 1]);
        packed[pp] = bits16(o0) | (bits16(o1) << 16);
      }
      __builtin_nontemporal_store(u32x4{packed[0], packed[1], packed[2], packed[3]},
                                  reinterpret_cast<u32x4*>(dst + row_out[tensor][row]));
    }
    // Block mean: combine the RPS row groups (lanes c, c+LPR, ...) in a fixed
    // butterfly order; the lanes of group 0 store the D means.
#pragma unroll
    for (int e = 0; e < 8; ++e) {
#pragma unroll
      for (int m = LPR; m < 64; m <<= 1) acc[e] += __shfl_xor(acc[e], m);
    }
    if (lane < LPR) {
      float* mp = a.mean[tensor] + ((int64_t)bh * a.nb + n) * D + 8 * c;
      constexpr float inv = 1.0f / 64.0f;
      *reinterpret_cast<float4*>(mp) = float4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
      *reinterpret_cast<float4*>(mp + 4) = float4{acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
    }
  }
}

template <typename T, int D>
hipError_t launch_prep_t(const PrepArgs& a, hipStream_t stream) {
  const size_t shmem = (size_t)a.table_len * sizeof(float);
  int dev = 0, cus = 0, per_cu = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e == hipSuccess)
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, prep_kernel<T, D>, 256, shmem);
  if (e != hipSuccess) return e;
  // As many workgroups as are resident at once (each stages the table once).
  const int want = (a.total_items + kPrepWaves - 1) / kPrepWaves;
  const int grid = std::max(1, std::min(want, cus * std::max(per_cu, 1)));
  hipLaunchKernelGGL((prep_kernel<T, D>), dim3(grid), dim3(256), shmem, stream, a);
  return hipGetLastError();
}

}  // namespace

bool prep_supported(int dtype, int D) { return dtype != 2 && (D == 64 || D == 128); }

hipError_t launch_prep(const Tensor4* in, const Tensor4* out, const void* const* weight,
                       float* const* mean, int dtype, int B, int H, int D, int nb, const Geom& g,
                       const int32_t* rope_grid, const int32_t* rope_dims, const float* table,
                       int table_len, float eps, hipStream_t stream) {
  PrepArgs a{};
  for (int t = 0; t < 2; ++t) {
    a.in[t] = in[t];
    a.out[t] = out[t];
    a.weight[t] = weight[t];
    a.mean[t] = mean[t];
  }
  a.table = table;
  a.H = H;
  a.D = D;
  a.nb = nb;
  a.rT = rope_grid[0];
  a.rH = rope_grid[1];
  a.rW = rope_grid[2];
  a.dt = rope_dims[0];
  a.dh = rope_dims[1];
  a.table_len = table_len;
  a.total_items = 2 * B * H * nb;
  a.eps = eps;
  a.g = g;
  a.per_block = make_fastdiv((uint32_t)(2 * B * H));
  a.heads = make_fastdiv((uint32_t)H);
  a.rcp_plane = (float)(1.0 / ((double)a.rH * a.rW));
  a.rcp_w = (float)(1.0 / (double)a.rW);
  a.neg_zero = -0.0f;
  a.one = 1.0f;
  if (dtype == 0) return D == 128 ? launch_prep_t<f16, 128>(a, stream) : launch_prep_t<f16, 64>(a, stream);
  return D == 128 ? launch_prep_t<bf16, 128>(a, stream) : launch_prep_t<bf16, 64>(a, stream);
}

}  // namespace lcv
