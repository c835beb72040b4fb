// Launch order of the q-blocks of each head for the attention kernel.
//
// Any order gives the same results up to fp32 rounding: each q-block is
// computed by one workgroup from its own routing list, and its launch slot
// sets where its walk over that list starts (the summation order).  For a
// given order the result is deterministic.  The order matters for the L2: each
// workgroup walks its KV blocks in ascending order, so workgroups that run at
// the same time on an XCD re-read each other's K/V tiles from L2 when their
// lists start at nearby blocks.  Sorting the q-blocks of a head by
// (first listed block, middle listed block) groups such lists; consecutive
// work ids land on the same XCD (xcd_linear_work_id), so the sorted runs
// execute together.
//
// q-block i's key is (first, median, i), with entries outside [0, nk) (the
// K/V block count of the head, which exceeds nq when keys outnumber queries)
// counting as nk.  The key is unique, so the sorted order is a permutation,
// the same one any correct sort gives.  Three sorts:
//   * nq <= 1024 and at most 512 workgroups of 64 keys: a rank sort, i to
//     position #{j : key_j < key_i}; each workgroup stages the head's keys
//     in LDS (32-bit when nq, nk <= 1023 fit 10 bits a field), and its four
//     waves count over a quarter of them each for the same 64 keys;
//   * other nq <= 1024: one workgroup per head, one key per thread, bitonic;
//     the stages whose partner lies in the same wave exchange keys with lane
//     shuffles, the rest through LDS;
//   * 1024 < nq <= 4096: a rank sort.  i goes to position #{j : key_j <
//     key_i}; every workgroup stages all keys of its head in LDS and ranks 256
//     of them, one per thread, in one pass over the staged keys (broadcast
//     LDS reads, no barriers after the staging), so a head's sort spreads
//     over ceil(nq / 256) workgroups instead of 78 dependent bitonic stages.
#include "bsa_common.h"

namespace lcv {
namespace {

constexpr int kMaxSched = 4096;
constexpr int kMaxKvBlocks = (1 << 20) - 1;  // a 20-bit key field holds 0 .. nk
constexpr int kRankThreads = 256;

// Sort key of q-block i: 20 bits each of its first and median list entries
// (out-of-range entries clamped to nk <= kMaxKvBlocks) and of i.
__device__ __forceinline__ uint64_t order_key(const int32_t* rows, int i, int nk, int top_k) {
  int first = rows[(int64_t)i * top_k];
  int median = rows[(int64_t)i * top_k + top_k / 2];
  first = (first < 0 || first >= nk) ? nk : first;
  median = (median < 0 || median >= nk) ? nk : median;
  return ((uint64_t)first << 40) | ((uint64_t)median << 20) | (uint64_t)i;
}

__global__ __launch_bounds__(kRankThreads) void schedule_rank_kernel(const int32_t* idx, int nq,
                                                                     int nk, int top_k,
                                                                     int32_t* order) {
  __shared__ uint64_t keys[kMaxSched];
  const int bh = blockIdx.x;
  const int32_t* rows = idx + (int64_t)bh * nq * top_k;
  for (int i = threadIdx.x; i < nq; i += kRankThreads) keys[i] = order_key(rows, i, nk, top_k);
  __syncthreads();
  const int i = blockIdx.y * kRankThreads + threadIdx.x;
  if (i >= nq) return;
  const uint64_t mine = keys[i];
  int rank = 0;
#pragma unroll 8
  for (int j = 0; j < nq; ++j) rank += keys[j] < mine ? 1 : 0;
  order[(int64_t)bh * nq + rank] = i;
}

// The bitonic sort for nq <= 1024 with one key per thread: the 45 of 55
// stages whose partner lies in the same wave (j < 64) exchange keys with lane
// shuffles; only the 10 with j >= 64 go through LDS and barriers.
constexpr int kSmallSched = 1024;

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t x, int m) {
  const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)x, m);
  const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(x >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

__global__ __launch_bounds__(kSmallSched) void schedule_small_kernel(const int32_t* idx, int nq,
                                                                     int nk, int top_k,
                                                                     int32_t* order) {
  __shared__ uint64_t xch[kSmallSched];
  const int bh = blockIdx.x;
  const int i = threadIdx.x;
  const int32_t* rows = idx + (int64_t)bh * nq * top_k;
  uint64_t key = i < nq ? order_key(rows, i, nk, top_k) : ~0ull;  // padding sorts last
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

// Rank sort for nq <= 1024 with the key packed into 32 bits when first,
// median (<= nk) and i fit 10 bits each, else 64.  A workgroup ranks 64 keys
// of one head: its four waves each count, for the same 64 keys (one per
// lane), the keys below them in a quarter of the head's staged keys
// (broadcast LDS reads), and the four partial ranks are summed.  A head's
// sort is spread over ceil(nq / 64) workgroups.
template <typename KeyT>
__device__ __forceinline__ KeyT pack_key(const int32_t* rows, int i, int nk, int top_k);
template <>
__device__ __forceinline__ uint32_t pack_key<uint32_t>(const int32_t* rows, int i, int nk, int top_k) {
  const uint64_t k = order_key(rows, i, nk, top_k);
  return (uint32_t)(((k >> 40) << 20) | (((k >> 20) & 0xFFFFFu) << 10) | (k & 0xFFFFFu));
}
template <>
__device__ __forceinline__ uint64_t pack_key<uint64_t>(const int32_t* rows, int i, int nk, int top_k) {
  return order_key(rows, i, nk, top_k);
}

constexpr int kRankGroup = 64;           // keys ranked per workgroup
constexpr int kRankSmallMaxWgs = 512;     // rank-sort grid limit (workgroups)

template <typename KeyT>
__global__ __launch_bounds__(256) void schedule_rank_small_kernel(const int32_t* idx, int nq, int nk,
                                                                  int top_k, int32_t* order) {
  __shared__ __attribute__((aligned(16))) KeyT keys[kSmallSched];
  __shared__ int part[4][kRankGroup];
  const int bh = blockIdx.x;
  const int tid = threadIdx.x;
  const int32_t* rows = idx + (int64_t)bh * nq * top_k;
  for (int i = tid; i < nq; i += 256) keys[i] = pack_key<KeyT>(rows, i, nk, top_k);
  __syncthreads();
  const int wave = tid / 64;
  const int lane = tid % 64;
  const int i = blockIdx.y * kRankGroup + lane;
  const KeyT mine = i < nq ? keys[i] : (KeyT)0;
  const int span = (nq + 3) / 4;
  const int j0 = wave * span;
  const int j1 = j0 + span < nq ? j0 + span : nq;
  int cnt = 0;
#pragma unroll 8
  for (int j = j0; j < j1; ++j) cnt += keys[j] < mine ? 1 : 0;
  part[wave][lane] = cnt;
  __syncthreads();
  if (wave == 0 && i < nq)
    order[(int64_t)bh * nq + (part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane])] = i;
}

}  // namespace

bool schedule_supported(int nq, int nk) {
  return nq >= 1 && nq <= kMaxSched && nk >= 1 && nk <= kMaxKvBlocks;
}

hipError_t launch_schedule(const int32_t* idx, int BH, int nq, int nk, int top_k, int32_t* order,
                           hipStream_t stream) {
  if (!schedule_supported(nq, nk) || BH < 1 || top_k < 1) return hipErrorInvalidValue;
  if (nq <= kSmallSched) {
    const int groups = (nq + kRankGroup - 1) / kRankGroup;
    // The rank sort stages every key of a head once per workgroup, so it
    // pays while the grid stays within about two workgroups per CU; larger
    // grids sort faster with the bitonic kernel.
    if ((int64_t)BH * groups <= kRankSmallMaxWgs) {
      const dim3 grid((unsigned)BH, (unsigned)groups);
      if (nk <= 1023)
        hipLaunchKernelGGL(schedule_rank_small_kernel<uint32_t>, grid, dim3(256), 0, stream, idx,
                           nq, nk, top_k, order);
      else
        hipLaunchKernelGGL(schedule_rank_small_kernel<uint64_t>, grid, dim3(256), 0, stream, idx,
                           nq, nk, top_k, order);
      return hipGetLastError();
    }
    hipLaunchKernelGGL(schedule_small_kernel, dim3(BH), dim3(kSmallSched), 0, stream, idx, nq, nk,
                       top_k, order);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)BH, (unsigned)((nq + kRankThreads - 1) / kRankThreads));
  hipLaunchKernelGGL(schedule_rank_kernel, grid, dim3(kRankThreads), 0, stream, idx, nq, nk, top_k,
                     order);
  return hipGetLastError();
}

}  // namespace lcv
