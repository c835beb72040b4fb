// Row operations of the DiT block around the attention, each one HBM pass:
//
//  * residual + LayerNorm: r = x, x + a, or x + gate * a (fp32, per-frame
//    gate), rounded to the tensor dtype; optionally written out; then
//    LayerNorm_FP32(r) with either the affine weight / bias or the AdaLN
//    modulation (* (scale + 1) + shift, per frame), rounded to the dtype
//    (longcat_video_dit.py:107-136 with blocks.py:79-119);
//  * SwiGLU gate: silu(a) * b over the two halves of the fused w1 / w3
//    projection (blocks.py:50-51);
//  * per-head RMSNorm_FP32 (blocks.py:55-72) from one layout to another, for
//    the cross-attention's q and k (attention.py:325-326).
//
// The reference runs each of these as several full-tensor passes in fp32.
#include <algorithm>

#include "norm_common.h"

namespace lcv {
namespace {

constexpr int kRowWaves = 4;

struct RowArgs {
  const void* x;
  const void* a;          // [rows, C] or null
  const float* gate;      // [B, T, C] or null: r = x + gate * a
  const float* shift;     // [B, T, C] or null: AdaLN modulation
  const float* scale;
  const void* ln_w;       // [C] in the tensor dtype or null: affine LayerNorm
  const void* ln_b;
  void* x_out;            // r, or null
  void* n_out;            // the normalised row, or null
  int32_t rows, C, rows_per_batch, tokens_per_frame, frames;
  float eps;
};

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* v) {
  const u32x4 raw = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    v[2 * m] = to_f32(__builtin_bit_cast(T, (uint16_t)(raw[m] & 0xffffu)));
    v[2 * m + 1] = to_f32(__builtin_bit_cast(T, (uint16_t)(raw[m] >> 16)));
  }
}

template <typename T>
__device__ __forceinline__ void store8(T* p, const float* v) {
  uint32_t w[4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
    w[m] = bits16(round_from_f32<T>(v[2 * m])) | (bits16(round_from_f32<T>(v[2 * m + 1])) << 16);
  *reinterpret_cast<u32x4*>(p) = u32x4{w[0], w[1], w[2], w[3]};
}

__device__ __forceinline__ void load8f(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
  v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}

// One wave per row; lane l holds the 8-element chunks l, l + 64, ... of the
// row (NMAX chunks at most, so C <= 512 * NMAX).
template <typename T, int NMAX>
__global__ __launch_bounds__(256) void rows_kernel(RowArgs p) {
  const int wave = uniform_i32(threadIdx.x / 64);
  const int lane = threadIdx.x % 64;
  const int row = blockIdx.x * kRowWaves + wave;
  if (row >= p.rows) return;  // wave-uniform
  const int b = row / p.rows_per_batch;
  const int t = (row - b * p.rows_per_batch) / p.tokens_per_frame;
  const int64_t frame = ((int64_t)b * p.frames + t) * p.C;
  const int64_t base = (int64_t)row * p.C;
  const int nch = p.C / 8;

  float r[NMAX][8];
#pragma unroll
  for (int i = 0; i < NMAX; ++i) {
    const int c = lane + 64 * i;
    if (c >= nch) break;
    load8(reinterpret_cast<const T*>(p.x) + base + 8 * c, r[i]);
    if (p.a) {
      float av[8];
      load8(reinterpret_cast<const T*>(p.a) + base + 8 * c, av);
      if (p.gate) {
        float g[8];
        load8f(p.gate + frame + 8 * c, g);
#pragma unroll
        for (int e = 0; e < 8; ++e) r[i][e] = to_f32(round_from_f32<T>(r[i][e] + g[e] * av[e]));
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) r[i][e] = to_f32(round_from_f32<T>(r[i][e] + av[e]));
      }
      if (p.x_out) store8(reinterpret_cast<T*>(p.x_out) + base + 8 * c, r[i]);
    }
  }
  if (!p.n_out) return;

  // LayerNorm in fp32: mean, then the mean of squared deviations.
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NMAX; ++i) {
    if (lane + 64 * i >= nch) break;
#pragma unroll
    for (int e = 0; e < 8; ++e) s += r[i][e];
  }
  const float mean = wave_sum(s) / (float)p.C;
  float q = 0.0f;
#pragma unroll
  for (int i = 0; i < NMAX; ++i) {
    if (lane + 64 * i >= nch) break;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float d = r[i][e] - mean;
      q += d * d;
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)p.C + p.eps);
#pragma unroll
  for (int i = 0; i < NMAX; ++i) {
    const int c = lane + 64 * i;
    if (c >= nch) break;
    float y[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) y[e] = (r[i][e] - mean) * rstd;
    if (p.ln_w) {
      float w[8], bb[8];
      load8(reinterpret_cast<const T*>(p.ln_w) + 8 * c, w);
      load8(reinterpret_cast<const T*>(p.ln_b) + 8 * c, bb);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = y[e] * w[e] + bb[e];
    }
    if (p.scale) {
      float sc[8], sh[8];
      load8f(p.scale + frame + 8 * c, sc);
      load8f(p.shift + frame + 8 * c, sh);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = y[e] * (sc[e] + 1.0f) + sh[e];
    }
    store8(reinterpret_cast<T*>(p.n_out) + base + 8 * c, y);
  }
}

template <typename T, int NMAX>
hipError_t launch_rows_t(const RowArgs& a, hipStream_t stream) {
  const int grid = (a.rows + kRowWaves - 1) / kRowWaves;
  hipLaunchKernelGGL((rows_kernel<T, NMAX>), dim3(grid), dim3(64 * kRowWaves), 0, stream, a);
  return hipGetLastError();
}

// silu(a) * b, each rounded to the dtype (torch's silu computes x / (1 +
// exp(-x)) in fp32; the product of two dtype values is exact in fp32).
template <typename T>
__global__ __launch_bounds__(256) void swiglu_kernel(const T* h, T* out, int64_t rows, int32_t hidden) {
  const int64_t n8 = rows * (hidden / 8);
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n8) return;
  const int64_t row = i / (hidden / 8);
  const int c = (int)(i - row * (hidden / 8));
  float a[8], bv[8], y[8];
  load8(h + row * 2 * hidden + 8 * c, a);
  load8(h + row * 2 * hidden + hidden + 8 * c, bv);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float s = to_f32(round_from_f32<T>(a[e] / (1.0f + expf(-a[e]))));
    y[e] = s * bv[e];
  }
  store8(out + row * hidden + 8 * c, y);
}

// RMSNorm_FP32 of rows of D elements: (b, n, h) -> out[b, h, n, :] (any
// strides), D / 8 lanes per row.
struct HeadNormArgs {
  const void* x;
  int64_t x_sb, x_sn, x_sh;
  void* out;
  int64_t o_sb, o_sn, o_sh;
  const void* w;  // [D] or null
  int32_t B, N, H, rows;
  float eps, neg_zero;
};

template <typename T, int D>
__global__ __launch_bounds__(256) void head_norm_kernel(HeadNormArgs p) {
  constexpr int LPR = D / 8;
  constexpr int RPW = 64 / LPR;  // rows per wave
  const int lane = threadIdx.x % 64;
  const int row = (blockIdx.x * 4 + (int)(threadIdx.x / 64)) * RPW + lane / LPR;
  const bool ok = row < p.rows;
  const int rr = ok ? row : 0;
  const int h = rr % p.H;
  const int bn = rr / p.H;
  const int n = bn % p.N;
  const int b = bn / p.N;
  const int c = lane % LPR;
  float x[8];
  load8(reinterpret_cast<const T*>(p.x) + b * p.x_sb + n * p.x_sn + h * p.x_sh + 8 * c, x);
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(x[e], x[e], ss);  // x*x exact in fp32
  ss = group_sum<LPR>(ss);
  const float rs = rsqrtf(ss * (1.0f / D) + p.eps);
  u32x4 wr;
  if (p.w) {
    wr = *reinterpret_cast<const u32x4*>(reinterpret_cast<const T*>(p.w) + 8 * c);
  } else {
    const uint32_t one = bits16(from_f32<T>(1.0f));
    wr = u32x4{one | (one << 16), one | (one << 16), one | (one << 16), one | (one << 16)};
  }
  float y[8];
  norm_scale<T>(x, rs, wr, p.neg_zero, y);
  if (ok) store8(reinterpret_cast<T*>(p.out) + b * p.o_sb + n * p.o_sn + h * p.o_sh + 8 * c, y);
}

}  // namespace

bool rows_supported(int dtype, int C) { return dtype != 2 && C > 0 && C % 8 == 0 && C <= 8192; }

hipError_t launch_rows(const void* x, const void* a, const float* gate, const float* shift,
                       const float* scale, const void* ln_w, const void* ln_b, void* x_out,
                       void* n_out, int dtype, int rows, int C, int rows_per_batch,
                       int tokens_per_frame, int frames, float eps, hipStream_t stream) {
  RowArgs p{x, a, gate, shift, scale, ln_w, ln_b, x_out, n_out,
            rows, C, rows_per_batch, tokens_per_frame, frames, eps};
  const int nmax = (C / 8 + 63) / 64;
  if (dtype == 0) {
    if (nmax <= 2) return launch_rows_t<f16, 2>(p, stream);
    if (nmax <= 8) return launch_rows_t<f16, 8>(p, stream);
    return launch_rows_t<f16, 16>(p, stream);
  }
  if (nmax <= 2) return launch_rows_t<bf16, 2>(p, stream);
  if (nmax <= 8) return launch_rows_t<bf16, 8>(p, stream);
  return launch_rows_t<bf16, 16>(p, stream);
}

hipError_t launch_swiglu(const void* h, void* out, int dtype, int64_t rows, int hidden,
                         hipStream_t stream) {
  const int64_t n8 = rows * (hidden / 8);
  const int grid = (int)((n8 + 255) / 256);
  if (dtype == 0)
    hipLaunchKernelGGL((swiglu_kernel<f16>), dim3(grid), dim3(256), 0, stream,
                       reinterpret_cast<const f16*>(h), reinterpret_cast<f16*>(out), rows, hidden);
  else
    hipLaunchKernelGGL((swiglu_kernel<bf16>), dim3(grid), dim3(256), 0, stream,
                       reinterpret_cast<const bf16*>(h), reinterpret_cast<bf16*>(out), rows, hidden);
  return hipGetLastError();
}

hipError_t launch_head_norm(const void* x, const int64_t* xs, void* out, const int64_t* os,
                            const void* w, int dtype, int B, int N, int H, int D, float eps,
                            hipStream_t stream) {
  HeadNormArgs p{x, xs[0], xs[1], xs[2], out, os[0], os[1], os[2], w, B, N, H, B * N * H, eps, -0.0f};
  const int rpw = 64 / (D / 8);
  const int grid = (p.rows + 4 * rpw - 1) / (4 * rpw);
  if (dtype == 0) {
    if (D == 128) hipLaunchKernelGGL((head_norm_kernel<f16, 128>), dim3(grid), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((head_norm_kernel<f16, 64>), dim3(grid), dim3(256), 0, stream, p);
  } else {
    if (D == 128) hipLaunchKernelGGL((head_norm_kernel<bf16, 128>), dim3(grid), dim3(256), 0, stream, p);
    else hipLaunchKernelGGL((head_norm_kernel<bf16, 64>), dim3(grid), dim3(256), 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace lcv
