// Block-mean pooling of q and k: [B,H,S,D] (t-major) -> [B,H,nb,D] fp32.
//
// Follows mean_pool_blocks_3d (longcat_video/models/block_sparse_attention.py:67-104):
// block n is a cT x cH x cW voxel of the (T, Hl, Wl) latent grid and its
// representative is the mean of the voxel's rows.  The reference reshapes and
// transposes the whole tensor first; here each wave walks the voxel's rows in
// place, so the only HBM traffic is one read of q and k and a small write.
//
// One wave per (tensor, b, h, block).  The D axis is split into 16-byte
// chunks (8 fp16/bf16 or 4 fp32 values); with D/VEC chunks per row, 64/(D/VEC)
// rows are in flight per load instruction.  Partial sums are combined through
// LDS in a fixed order, so results are deterministic.
#include "bsa_common.h"

namespace lcv {
namespace {

constexpr int kWavesPerWg = 4;

// Raw 16-byte (or one-element) loads and their accumulation, split so that
// several rows' loads can be in flight before any of them is added.
template <typename T, int VEC>
struct VecLoad;

template <typename T>
struct VecLoad<T, 8> {  // 8 x 16-bit
  typedef u32x4 Raw;
  // Non-temporal: q and k are read once here (5.35 -> 5.75 TB/s for the
  // 944 MB of the 720p shape).
  __device__ static Raw load(const T* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  }
  __device__ static void add(const Raw& w, float* acc) {
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      acc[2 * m] += to_f32(__builtin_bit_cast(T, (uint16_t)(w[m] & 0xffffu)));
      acc[2 * m + 1] += to_f32(__builtin_bit_cast(T, (uint16_t)(w[m] >> 16)));
    }
  }
};

template <>
struct VecLoad<float, 4> {
  typedef f32x4 Raw;
  __device__ static Raw load(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
  __device__ static void add(const Raw& w, float* acc) {
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] += w[m];
  }
};

template <typename T>
struct VecLoad<T, 1> {
  typedef T Raw;
  __device__ static Raw load(const T* p) { return *p; }
  __device__ static void add(const Raw& w, float* acc) { acc[0] += to_f32(w); }
};

constexpr int kRowTable = 256;  // voxel rows whose offsets are tabulated in LDS
constexpr int kBatch = 8;       // row loads in flight per lane

struct PoolArgs {
  Tensor4 x[2];
  float* out[2];
  int32_t B, H, D, nb, bs;
  int32_t items_per_tensor;
  int32_t total_items;
  Geom g;
};

template <typename T, int VEC>
__global__ __launch_bounds__(256) void pool_kernel(PoolArgs a) {
  __shared__ float part[kWavesPerWg][64 * VEC];
  __shared__ int32_t row_off[kRowTable];
  // Token offset of each voxel row from the block's first token: the same
  // for every block, so computed once per workgroup.
  const bool table = a.bs <= kRowTable;
  if (table)
    for (int r = threadIdx.x; r < a.bs; r += blockDim.x) row_off[r] = voxel_row_offset(a.g, r);
  __syncthreads();
  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  const int item_raw = blockIdx.x * kWavesPerWg + wave;
  // Waves past the end still take part in the barriers below.
  const bool valid = item_raw < a.total_items;
  const int item = valid ? item_raw : 0;

  const int t = item / a.items_per_tensor;
  const int rem = item - t * a.items_per_tensor;
  const int bh = rem / a.nb;
  const int n = rem - bh * a.nb;
  const int b = bh / a.H;
  const int h = bh - b * a.H;

  const Tensor4 x = a.x[t];
  const T* base = reinterpret_cast<const T*>(x.ptr) + (int64_t)b * x.sb + (int64_t)h * x.sh;
  const int32_t tok0 = block_base_token(a.g, n);
  float* out = a.out[t] + ((int64_t)bh * a.nb + n) * a.D;
  const int DC = a.D / VEC;  // chunks per row
  const float inv_bs = 1.0f / (float)a.bs;

  for (int c0 = 0; c0 < DC; c0 += 64) {
    const int cols = (DC - c0) < 64 ? (DC - c0) : 64;
    const int P = 64 / cols;  // rows in flight per instruction
    const int c = c0 + lane % cols;
    const int p = lane / cols;
    float acc[VEC];
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
    if (valid && p < P) {
      typedef VecLoad<T, VEC> L;
      const T* col = base + c * VEC;
      // Rows p, p + P, p + 2P, ... are added in this order either way; the
      // batches only put kBatch loads in flight before the adds.
      int r = p;
      if (table) {
        for (; r + (kBatch - 1) * P < a.bs; r += kBatch * P) {
          typename L::Raw w[kBatch];
#pragma unroll
          for (int u = 0; u < kBatch; ++u)
            w[u] = L::load(col + (int64_t)(tok0 + row_off[r + u * P]) * x.ss);
          // Keep the scheduler from pairing each load with its add.
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int u = 0; u < kBatch; ++u) L::add(w[u], acc);
        }
      }
      for (; r < a.bs; r += P)
        L::add(L::load(col + (int64_t)(tok0 + voxel_row_offset(a.g, r)) * x.ss), acc);
    }
    // Combine the P partial sums of each column chunk in phase order.
#pragma unroll
    for (int e = 0; e < VEC; ++e) part[wave][lane * VEC + e] = acc[e];
    __syncthreads();
    for (int o = lane; valid && o < cols * VEC; o += 64) {
      const int cc = o / VEC;  // chunk within this group
      const int e = o - cc * VEC;
      float s = 0.0f;
      for (int q = 0; q < P; ++q) s += part[wave][(q * cols + cc) * VEC + e];
      out[(c0 + cc) * VEC + e] = s * inv_bs;
    }
    __syncthreads();
  }
}

template <typename T, int VEC>
hipError_t launch_pool_t(const PoolArgs& a, hipStream_t stream) {
  const int grid = (a.total_items + kWavesPerWg - 1) / kWavesPerWg;
  hipLaunchKernelGGL((pool_kernel<T, VEC>), dim3(grid), dim3(64 * kWavesPerWg), 0, stream, a);
  return hipGetLastError();
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

hipError_t launch_pool(const Tensor4* xs, int n_tensors, int dtype, int B, int H, int D,
                       int nb, int bs, const Geom& g, float* const* outs,
                       hipStream_t stream) {
  PoolArgs a{};
  for (int t = 0; t < n_tensors; ++t) {
    a.x[t] = xs[t];
    a.out[t] = outs[t];
  }
  a.B = B;
  a.H = H;
  a.D = D;
  a.nb = nb;
  a.bs = bs;
  a.items_per_tensor = B * H * nb;
  a.total_items = a.items_per_tensor * n_tensors;
  a.g = g;

  const int elem = dtype == LCV_BSA_F32 ? 4 : 2;
  const int vec = 16 / elem;
  bool vec_ok = (D % vec) == 0;
  for (int t = 0; t < n_tensors; ++t) {
    vec_ok = vec_ok && aligned16(xs[t].ptr) && (xs[t].sb % vec) == 0 &&
             (xs[t].sh % vec) == 0 && (xs[t].ss % vec) == 0;
  }
  switch (dtype) {
    case LCV_BSA_F16:
      return vec_ok ? launch_pool_t<f16, 8>(a, stream) : launch_pool_t<f16, 1>(a, stream);
    case LCV_BSA_BF16:
      return vec_ok ? launch_pool_t<bf16, 8>(a, stream) : launch_pool_t<bf16, 1>(a, stream);
    default:
      return vec_ok ? launch_pool_t<float, 4>(a, stream) : launch_pool_t<float, 1>(a, stream);
  }
}

}  // namespace lcv
