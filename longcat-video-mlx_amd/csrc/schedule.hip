// Launch order of the q-blocks of each head for the attention kernel.
//
// Any order gives bit-identical results (each q-block is computed by one
// workgroup from its own routing list).  The order matters for the L2: each
// workgroup walks its KV blocks in ascending order, so workgroups that run at
// the same time on an XCD re-read each other's K/V tiles from L2 when their
// lists start at nearby blocks.  Sorting the q-blocks of a head by
// (first listed block, middle listed block) groups such lists; consecutive
// work ids land on the same XCD (xcd_linear_work_id), so the sorted runs
// execute together.
//
// One workgroup per (b, h): keys are built from idx[b,h,i,0] and
// idx[b,h,i,top_k/2] (entries outside [0, nq) count as nq) and bitonic-sorted
// in LDS together with the q-block index, which also makes the order a
// permutation.
#include "bsa_common.h"

namespace lcv {
namespace {

constexpr int kMaxSched = 4096;

__global__ __launch_bounds__(256) void schedule_kernel(const int32_t* idx, int nq, int top_k,
                                                       int n_pow2, int32_t* order) {
  __shared__ uint64_t keys[kMaxSched];
  const int bh = blockIdx.x;
  const int32_t* rows = idx + (int64_t)bh * nq * top_k;
  const int mid = top_k / 2;
  for (int i = threadIdx.x; i < n_pow2; i += 256) {
    uint64_t key = ~0ull;  // padding sorts last
    if (i < nq) {
      int first = rows[(int64_t)i * top_k];
      int median = rows[(int64_t)i * top_k + mid];
      first = (first < 0 || first >= nq) ? nq : first;
      median = (median < 0 || median >= nq) ? nq : median;
      key = ((uint64_t)first << 40) | ((uint64_t)median << 20) | (uint64_t)i;
    }
    keys[i] = key;
  }
  __syncthreads();
  for (int k = 2; k <= n_pow2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n_pow2; i += 256) {
        const int p = i ^ j;
        if (p > i) {
          const uint64_t a = keys[i], b = keys[p];
          const bool up = (i & k) == 0;
          if ((a > b) == up) {
            keys[i] = b;
            keys[p] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  for (int i = threadIdx.x; i < nq; i += 256)
    order[(int64_t)bh * nq + i] = (int32_t)(keys[i] & 0xFFFFFu);
}

// The same sort for nq <= 1024 with one key per thread: the 45 of 55
// bitonic stages whose partner lies in the same wave (j < 64) exchange keys
// with lane shuffles; only the 10 with j >= 64 go through LDS and barriers.
constexpr int kSmallSched = 1024;

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)x, m);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

__global__ __launch_bounds__(kSmallSched) void schedule_small_kernel(const int32_t* idx, int nq,
                                                                     int top_k, int32_t* order) {
  __shared__ uint64_t xch[kSmallSched];
  const int bh = blockIdx.x;
  const int i = threadIdx.x;
  const int32_t* rows = idx + (int64_t)bh * nq * top_k;
  const int mid = top_k / 2;
  uint64_t key = ~0ull;  // padding sorts last
  if (i < nq) {
    int first = rows[(int64_t)i * top_k];
    int median = rows[(int64_t)i * top_k + mid];
    first = (first < 0 || first >= nq) ? nq : first;
    median = (median < 0 || median >= nq) ? nq : median;
    key = ((uint64_t)first << 40) | ((uint64_t)median << 20) | (uint64_t)i;
  }
  for (int k = 2; k <= kSmallSched; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      uint64_t other;
      if (j < 64) {
        other = shfl_xor_u64(key, j);
      } else {
        xch[i] = key;
        __syncthreads();
        other = xch[i ^ j];
        __syncthreads();
      }
      const bool up = (i & k) == 0;
      const bool lower = (i & j) == 0;  // i < i ^ j
      const uint64_t lo = other < key ? other : key;
      const uint64_t hi = other < key ? key : other;
      key = (lower == up) ? lo : hi;
    }
  }
  if (i < nq) order[(int64_t)bh * nq + i] = (int32_t)(key & 0xFFFFFu);
}

}  // namespace

bool schedule_supported(int nq) { return nq >= 1 && nq <= kMaxSched; }

hipError_t launch_schedule(const int32_t* idx, int BH, int nq, int top_k, int32_t* order,
                           hipStream_t stream) {
  if (nq <= kSmallSched) {
    hipLaunchKernelGGL(schedule_small_kernel, dim3(BH), dim3(kSmallSched), 0, stream, idx, nq,
                       top_k, order);
    return hipGetLastError();
  }
  int n = 1;
  while (n < nq) n <<= 1;
  hipLaunchKernelGGL(schedule_kernel, dim3(BH), dim3(256), 0, stream, idx, nq, top_k, n, order);
  return hipGetLastError();
}

}  // namespace lcv
