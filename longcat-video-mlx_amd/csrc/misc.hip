// Index and layout helpers of the block sparse attention path: the token ->
// block map, the token-pair mask and the t-major <-> block-major permutation.
// They are integer / copy kernels; the attention kernels never need them
// (they address voxel rows directly), but they reproduce the reference's
// helpers bit for bit.
#include "bsa_common.h"

namespace lcv {
namespace {

// Block of token s: build_token_block_indices,
// longcat_video/models/block_sparse_attention.py:137-159.
__device__ __forceinline__ int32_t block_of_token(const Geom& g, int32_t s) {
  const int32_t t = s / g.HW;
  const int32_t hw = s - t * g.HW;
  const int32_t hh = hw / g.Wl;
  const int32_t w = hw - hh * g.Wl;
  return (t / g.cT) * (g.Bh * g.Bw) + (hh / g.cH) * g.Bw + w / g.cW;
}

__global__ void token_blocks_kernel(Geom g, int32_t S, int32_t* out) {
  const int32_t s = blockIdx.x * blockDim.x + threadIdx.x;
  if (s < S) out[s] = block_of_token(g, s);
}

// build_token_pair_mask, block_sparse_attention.py:162-198: one thread per
// (b, h, sq, sk).  A token whose block falls outside [0, nq) gets an all-zero
// row (never read out of bounds).
__global__ void pair_mask_kernel(const int32_t* idx, int32_t nq, int32_t top_k,
                                 const int32_t* token_block, int32_t S, int32_t nkv,
                                 int64_t total, uint8_t* mask) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int64_t SS = (int64_t)S * S;
  const int64_t bh = e / SS;
  const int64_t rem = e - bh * SS;
  const int32_t sq = (int32_t)(rem / S);
  const int32_t sk = (int32_t)(rem - (int64_t)sq * S);
  const int32_t qb = token_block[sq];
  const int32_t kb = token_block[sk];
  uint8_t hit = 0;
  if (qb >= 0 && qb < nq && kb >= 0 && kb < nkv) {
    const int32_t* list = idx + (bh * nq + qb) * top_k;
    for (int32_t j = 0; j < top_k; ++j) hit |= (uint8_t)(list[j] == kb);
  }
  mask[e] = hit;
}

// _reshape_to_block_major / _reshape_from_block_major,
// longcat_video/models/block_sparse_attention_metal.py:185-221.  One thread per
// element (elements of 2 or 4 bytes).
template <typename E>
__global__ void permute_kernel(const E* x, int32_t S, int32_t D, int32_t bs, int64_t total,
                               Geom g, int inverse, E* out) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= total) return;
  const int64_t SD = (int64_t)S * D;
  const int64_t bh = e / SD;
  const int64_t rem = e - bh * SD;
  const int32_t row = (int32_t)(rem / D);  // block-major row
  const int32_t d = (int32_t)(rem - (int64_t)row * D);
  const int32_t n = row / bs;
  const int32_t r = row - n * bs;
  const int32_t tok = block_base_token(g, n) + voxel_row_offset(g, r);
  const int64_t bm = bh * SD + (int64_t)row * D + d;
  const int64_t tm = bh * SD + (int64_t)tok * D + d;
  if (inverse)
    out[tm] = x[bm];
  else
    out[bm] = x[tm];
}

}  // namespace

hipError_t launch_token_blocks(const Geom& g, int T, int32_t* out, hipStream_t stream) {
  const int32_t S = T * g.HW;
  hipLaunchKernelGGL(token_blocks_kernel, dim3((S + 255) / 256), dim3(256), 0, stream, g, S, out);
  return hipGetLastError();
}

hipError_t launch_pair_mask(const int32_t* idx, int B, int H, int nq, int top_k,
                            const int32_t* token_block, int S, int nkv, uint8_t* mask,
                            hipStream_t stream) {
  const int64_t total = (int64_t)B * H * S * S;
  const int64_t grid = (total + 255) / 256;
  hipLaunchKernelGGL(pair_mask_kernel, dim3((unsigned)grid), dim3(256), 0, stream, idx, nq, top_k,
                     token_block, S, nkv, total, mask);
  return hipGetLastError();
}

hipError_t launch_permute(const void* x, int elem_bytes, int B, int H, int S, int D,
                          const Geom& g, int inverse, void* out, hipStream_t stream) {
  const int64_t total = (int64_t)B * H * S * D;
  const int64_t grid = (total + 255) / 256;
  const int bs = g.cT * g.cH * g.cW;
  if (elem_bytes == 2) {
    hipLaunchKernelGGL(permute_kernel<uint16_t>, dim3((unsigned)grid), dim3(256), 0, stream,
                       reinterpret_cast<const uint16_t*>(x), S, D, bs, total, g, inverse,
                       reinterpret_cast<uint16_t*>(out));
  } else {
    hipLaunchKernelGGL(permute_kernel<uint32_t>, dim3((unsigned)grid), dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(x), S, D, bs, total, g, inverse,
                       reinterpret_cast<uint32_t*>(out));
  }
  return hipGetLastError();
}

}  // namespace lcv
