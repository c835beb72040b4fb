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
// MFMA kernel (fp16 / bf16, sm_scale >= 0, D = 64 or 128): attn_half_kernel.
//   * one workgroup (2 waves) per (b, h, q-block); wave w owns query rows
//     32w..32w+31 of the block; three (D = 128) or four (D = 64) waves per
//     SIMD are resident, so one wave's softmax overlaps another's MFMAs;
//   * each listed 64-key block is processed as two 32-key halves on
//     16 x 16 x 32 MFMAs (fp32 accumulate); the wave's Q tile stays in
//     registers as the B operand of S^T = K Q^T, and S^T's accumulator layout
//     is the B-operand layout of O^T = V^T P^T after a fixed relabelling of
//     the keys, so P never leaves registers;
//   * the exponent offset m of a row is the max of its first half; later
//     halves compute P = exp2(s*scale*log2e - m) without a max pass; P is
//     rounded once, and its rounded copy feeds both the PV product and the
//     row sum (v_dot2), so numerator and denominator agree; a half whose P sum
//     would pass 2^15 sends the workgroup through an exact second walk;
//   * K and V half tiles go from HBM straight into a three-slot LDS ring with
//     buffer_load ... lds (no register staging), row-major with 16-byte chunks
//     XOR-swizzled by row so that every operand read is bank-conflict free:
//     K rows are read with ds_read_b128, V^T operands with ds_read_b64_tr_b16
//     (lane L of a 16-lane group receives element L%4 of the rows read by
//     lanes L/4 + {0,4,8,12}, i.e. 4 consecutive keys of one V column);
//   * every half tile is fetched two ring elements ahead (explicit vmcnt
//     waits); workgroups are ordered so each XCD sweeps the q-blocks of one
//     head (shared K/V in its L2), and each workgroup starts its ascending
//     list at a block index set by its launch slot, so the workgroups resident
//     on an XCD walk a narrow window of K/V blocks together;
//   * the routing list is read 64 entries at a time; each lane turns its entry
//     into the block's first token once, so a block costs one v_readlane;
//   * the output tile is staged through LDS and written as whole rows.
//
// Vector-ALU kernel (any dtype, D in {16, 32, 64, 128, 256}, any scale): 64
// rows x 4 lanes per workgroup, fp32 throughout; used for fp32 inputs, head
// dims without an MFMA tiling and negative scales.
#include "bsa_common.h"

namespace lcv {
namespace {

// MFMA kernel: bound on a half tile's partial sum of P values, so that every
// P stays <= 2^15, a normal fp16 value.  Past it the workgroup walks again
// with the exact row maxima.
constexpr float kMaxTileSum = 32768.0f;
constexpr int kBufferFlags = 0x00020000;  // raw buffer, 32-bit dwords (gfx9 family)

typedef __attribute__((address_space(3))) void lds_void;
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// NaN-propagating max of three (v_maximum3_f32).
__device__ __forceinline__ float fmax3(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// Lanes l and l ^ 32 exchange x through v_permlane32_swap (a VALU op; no
// LDS round trip); the two results hold x[l] and x[l ^ 32] in some order.
__device__ __forceinline__ void swap_halves(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, x), false, false);
  a = __builtin_bit_cast(float, (uint32_t)r[0]);
  b = __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ __forceinline__ float max_halves(float x) {
  float a, b;
  swap_halves(x, a, b);
  return __builtin_elementwise_maximum(a, b);
}
__device__ __forceinline__ float sum_halves(float x) {
  float a, b;
  swap_halves(x, a, b);
  return a + b;
}

__device__ __forceinline__ int next_valid(const int32_t* list, int j, int top_k, int nb) {
  while (j < top_k) {
    const int n = uniform_i32(list[j]);
    if (n >= 0 && n < nb) break;
    ++j;
  }
  return j;
}

// A q-block's routing list, read 64 entries at a time into one register:
// lane l holds the first token of block list[base + l] (-1 if the entry is
// outside [0, nb)), computed once per chunk with vector ops, plus a wave mask
// of the valid entries.  The tile loop then needs one v_readlane per tile
// and issues no vector loads of its own between tile fetches.
struct TileList {
  const int32_t* list;
  int top_k, nb, base;
  int raw;         // per lane: list entry base + l (INT_MAX past top_k)
  int tok;         // per lane
  uint64_t valid;  // bit l: entry base + l is a block in [0, nb)
  // Issues the load of entries 0..63; finish() converts them once they are
  // needed, so other loads can be in flight meanwhile.
  __device__ TileList(const int32_t* l, int k, int n) : list(l), top_k(k), nb(n), base(0) {
    raw = fetch(0);
  }
  __device__ int fetch(int b) const {
    const int j = b + lane_id();
    return j < top_k ? list[j] : 0x7fffffff;
  }
  __device__ void finish(const Geom& g) {
    const bool ok = raw >= 0 && raw < nb;
    tok = ok ? block_base_token(g, raw) : -1;
    valid = __ballot(ok);
  }
  __device__ void load(int b, const Geom& g) {
    base = b;
    raw = fetch(b);
    finish(g);
  }
  // First j' >= j whose entry is valid, or top_k.  j uniform.
  __device__ int next(int j, const Geom& g) {
    while (j < top_k) {
      if (j < base || j - base >= 64) load(j & ~63, g);
      const uint64_t m = valid >> (j - base);
      if (m) return j + (int)__builtin_ctzll(m);
      j = base + 64;
    }
    return top_k;
  }
  // First token of entry j (valid, within the current chunk).
  __device__ int32_t token(int j) const { return __builtin_amdgcn_readlane(tok, j - base); }
  // Number of entries before the first one >= n0 in an ascending list (for
  // any list: the count of leading entries < n0, which is a valid start).
  // Called with the first chunk in place; a one-chunk list needs no load.
  __device__ int count_below(int n0, const Geom& g) {
    int cnt = __popcll(__ballot(raw < n0));
    if (cnt < 64 || top_k <= 64) return cnt;
    for (int b = 64; b < top_k; b += 64) {
      load(b, g);
      const int c = __popcll(__ballot(raw < n0));
      cnt += c;
      if (c < 64) break;
    }
    return cnt;
  }
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// 16 bytes per lane from a raw buffer straight into LDS: lane i writes
// lds_dst + 16 i (1 KB per wave).  Issued as inline asm so that the only
// waits on it are the explicit wait_vmcnt<> calls (the compiler otherwise
// waits for every outstanding LDS load before any LDS read).
// The immediate OFF is added to both the memory and the LDS address, so four
// loads 1 KB apart in LDS share one M0 value when each lane's voffset is
// pre-reduced by OFF (the memory offset of a load's rows is at least OFF).
template <int OFF>
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, int32_t soffset,
                                      uint32_t m0v) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen offset:%3 lds"
               ::"v"(voffset), "s"(rsrc), "s"(soffset), "i"(OFF), "{m0}"(m0v)
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

template <typename T>
struct Mfma;

template <>
struct Mfma<f16> {
  typedef f16x8 vec8;
  typedef _Float16 vec2 __attribute__((ext_vector_type(2)));
  __device__ static f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  // Sum of the 8 elements of v added to acc.
  __device__ static float sum8(vec8 v, float acc) {
    const vec2 one = {(f16)1.0f, (f16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const vec2 pr = {v[2 * i], v[2 * i + 1]};
      acc = __builtin_amdgcn_fdot2(pr, one, acc, false);
    }
    return acc;
  }
};

template <>
struct Mfma<bf16> {
  typedef bf16x8 vec8;
  typedef __bf16 vec2 __attribute__((ext_vector_type(2)));
  __device__ static f32x4 mma(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static float sum8(vec8 v, float acc) {
    const vec2 one = {(bf16)1.0f, (bf16)1.0f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const vec2 pr = {v[2 * i], v[2 * i + 1]};
      acc = __builtin_amdgcn_fdot2_f32_bf16(pr, one, acc, false);
    }
    return acc;
  }
};

// Tile geometry.  K and V rows are row-major in LDS, 2*D bytes per row,
// DC = D/8 16-byte chunks per row.  Chunk c of row r is stored at chunk
// position c ^ swz(r):
//   K: swz = (r / RP) % DC          -- 16 rows read one chunk column: conflict free
//   V: swz = 2 * ((r / RP) % (DC/2)) -- 8 rows x 32 bytes per 32-lane tr-read: conflict free
// where RP = 256 / (2*D) rows share one 256-byte bank span.
template <typename T, int D>
struct MfmaCfg {
  static constexpr int kThreads = 128;
  static constexpr int DC = D / 8;
  static constexpr int RP = 256 / (2 * D);
  static constexpr int kRowsPerDma = 64 / DC;  // rows per 1 KB wave load
  static_assert(D == 64 || D == 128, "MFMA tiling covers D = 64, 128");
  __device__ static int kswz(int r) { return (r / RP) % DC; }
  __device__ static int vswz(int r) { return 2 * ((r / RP) % (DC / 2)); }
};

// ---------------------------------------------------------------------------
// Half-block MFMA kernel (fp16 / bf16, D = 64 or 128).  One workgroup of 2
// waves per (b, h, q-block), wave w owns query rows 32w .. 32w + 31; each
// listed 64-key block is processed as two 32-key halves, one after the other,
// and both products run on 16 x 16 x 32 MFMAs.  Per wave and half:
//   S^T[kt][qt] (16 keys x 16 queries) += K[kt] (16 x 32 of D) Q^T[qt] over
//     D / 32 D steps; lane l holds query 16 qt + l % 16 and keys
//     16 kt + 4 (l / 16) + i;
//   O^T[dt][qt] (16 of D x 16 queries) += V^T[dt] (16 x 32 keys) P^T[qt],
//     dt < D / 16.  P^T stays in registers as the B operand: its contraction
//     index 8 (l / 16) + j stands for key 16 (j / 4) + 4 (l / 16) + j % 4,
//     and the V^T operand is read from LDS in the same key order.
// The 16 x 16 form reads a fifth fewer operand registers per FLOP than
// 32 x 32 x 16, and on this power-limited chip that is time.  Each query's
// keys sit in four lane groups (l, l ^ 16, l ^ 32, l ^ 48): the row max and
// the final row sum reduce over all four (v_permlane16_swap, then
// v_permlane32_swap).  A wave's state (Q, O, S 16 and P 8 registers) fits 168
// registers at D = 128 (three waves per SIMD) and 112 at D = 64 (four).
//
// The K and V half tiles (32 rows each) flow through a ring of three LDS
// slots, 24 KB per workgroup at D = 128: six workgroups per CU (eight at
// D = 64).  Ring order, per block: K(lo), V(lo), K(hi), V(hi).  Element e of
// that sequence sits in slot e mod 3.  At the barrier that starts element e,
// both waves have consumed element e - 1 and waited for their halves of e,
// so the DMA of element e + 2 goes into e - 1's slot: every half tile is
// fetched two elements ahead, with one barrier per element.  Each workgroup
// starts its ascending list at the first entry at or above a block index set
// by its launch slot (the sweep start, below), so that the workgroups
// resident on an XCD walk one window of K/V blocks together.
// ---------------------------------------------------------------------------
template <int N>
struct Phase {
  static constexpr int value = N;
};

// Lanes l and l ^ 16 exchange x through v_permlane16_swap; the two results
// hold x[l] and x[l ^ 16] in some order.
__device__ __forceinline__ void swap_rows16(float x, float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, x), false, false);
  a = __builtin_bit_cast(float, (uint32_t)r[0]);
  b = __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ __forceinline__ float max_quarters(float x) {
  float a, b;
  swap_rows16(x, a, b);
  return max_halves(__builtin_elementwise_maximum(a, b));
}
__device__ __forceinline__ float sum_quarters(float x) {
  float a, b;
  swap_rows16(x, a, b);
  return sum_halves(a + b);
}

// Waves per SIMD for attn_half_kernel: D = 128 holds 168 registers per wave,
// D = 64 (half the Q and O state) 128.
template <int D>
struct HalfOccupancy {
  static constexpr int kWaves = D == 128 ? 3 : 4;
};

template <typename T, int D>
__global__ __launch_bounds__(128)
__attribute__((amdgpu_waves_per_eu(HalfOccupancy<D>::kWaves, HalfOccupancy<D>::kWaves)))
void attn_half_kernel(AttnParams p) {
  static_assert(D == 64 || D == 128, "half-block tiling covers D = 64, 128");
  typedef MfmaCfg<T, D> C;
  typedef typename Mfma<T>::vec8 vec8;
  constexpr int kSlotBytes = 32 * 2 * D;  // 32 rows of K or V: 8 KB at D = 128
  constexpr int kGroup = 16 * 2 * D;      // bytes of 16 rows: the second key tile / key group
  constexpr int kLoads = kSlotBytes / 1024 / 2;  // 1 KB DMA loads per wave per half tile
  __shared__ __attribute__((aligned(1024))) uint8_t ring[3 * kSlotBytes];

  const int wid = xcd_linear_work_id(blockIdx.x, gridDim.x);
  const int bh = wid / p.nb;
  const int qb = p.order ? uniform_i32(p.order[wid]) : wid - bh * p.nb;
  if ((uint32_t)qb >= (uint32_t)p.nb) return;  // a launch-order entry outside [0, nb): nothing to do
  const int b = bh / p.H;
  const int h = bh - b * p.H;
  const int tid = threadIdx.x;
  const int wave = uniform_i32(tid / 64);
  const int lane = tid % 64;
  const int G = lane / 16;   // lane group: keys 4G.. of each 16-key tile, D rows 4G.. of O
  const int gi = lane % 16;  // query 16 qt + gi

  const T* qbase = reinterpret_cast<const T*>(p.q) + (int64_t)b * p.q_sb + (int64_t)h * p.q_sh;
  const T* kbase = reinterpret_cast<const T*>(p.k) + (int64_t)b * p.k_sb + (int64_t)h * p.k_sh;
  const T* vbase = reinterpret_cast<const T*>(p.v) + (int64_t)b * p.v_sb + (int64_t)h * p.v_sh;
  T* obase = reinterpret_cast<T*>(p.out) + (int64_t)b * p.o_sb + (int64_t)h * p.o_sh;
  const __amdgpu_buffer_rsrc_t krs =
      __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, (int)p.k_head_bytes, kBufferFlags);
  const __amdgpu_buffer_rsrc_t vrs =
      __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, (int)p.v_head_bytes, kBufferFlags);

  TileList list(p.idx + ((int64_t)bh * p.nb + qb) * p.top_k, p.top_k, p.nk);

  // Q^T operand: qf[qt][ks] holds query 32 wave + 16 qt + gi, D 32 ks + 8 G .. + 7.
  // Q is read once and O written once per launch: both go non-temporal, so
  // that they do not evict the K/V tiles other workgroups re-read from L2
  // (-0.5 to -0.9 % kernel time at 28,800-115,200 q-blocks, same bits).
  vec8 qf[2][D / 32];
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const int32_t qtok = block_base_token(p.g, qb) + voxel_row_offset(p.g, 32 * wave + 16 * qt + gi);
    const T* qrow = qbase + (int64_t)qtok * p.q_ss + 8 * G;
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
      qf[qt][ks] = __builtin_bit_cast(vec8, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(qrow + 32 * ks)));
  }
  list.finish(p.gk);

  // ---- DMA: a half tile is 32 rows (2 kLoads wave loads of 1 KB); wave w
  // loads rows 16w .. 16w + 15 of it (kLoads loads).  Row r + 32 of a block
  // sits voxel_row_offset(32) tokens after row r (voxel sides are powers of
  // two), so the high half uses the low half's lane offsets plus a scalar.
  uint32_t kvo[kLoads], vvo[kLoads];
#pragma unroll
  for (int u = 0; u < kLoads; ++u) {
    const int t = kLoads * wave + u;
    const int row = t * C::kRowsPerDma + lane / C::DC;  // 0 .. 31
    const int pc = lane % C::DC;
    const uint32_t tokoff = (uint32_t)voxel_row_offset(p.gk, row);
    kvo[u] = (tokoff * (uint32_t)p.k_ss + 8u * (pc ^ C::kswz(row))) * sizeof(T) - 1024u * u;
    vvo[u] = (tokoff * (uint32_t)p.v_ss + 8u * (pc ^ C::vswz(row))) * sizeof(T) - 1024u * u;
  }
  const uint32_t k_row_bytes = (uint32_t)p.k_ss * sizeof(T);
  const uint32_t v_row_bytes = (uint32_t)p.v_ss * sizeof(T);
  const uint32_t hi_tok = (uint32_t)voxel_row_offset(p.gk, 32);
  auto dma = [&](int32_t tok, int half, int isv, int slot) {
    const uint32_t t = (uint32_t)tok + (half ? hi_tok : 0u);
    const uint32_t m0v = lds_addr(ring + slot * kSlotBytes + 1024 * (kLoads * wave));
    const __amdgpu_buffer_rsrc_t rs = isv ? vrs : krs;
    const uint32_t* vo = isv ? vvo : kvo;
    const int off = (int)(t * (isv ? v_row_bytes : k_row_bytes));
    dma16<0>(rs, vo[0], off, m0v);
    dma16<1024>(rs, vo[1], off, m0v);
    if constexpr (kLoads == 4) {
      dma16<2048>(rs, vo[2], off, m0v);
      dma16<3072>(rs, vo[3], off, m0v);
    }
  };

  // LDS operand addresses.  K[kt] for D step ks: row 16 kt + gi (kt adds
  // kGroup bytes), chunk 4 ks + G.  V^T[dt]: rows 4 G .. 4 G + 3 (+ 16 for
  // the second key group, kGroup further), columns 16 dt + 4 (gi % 4) .. + 3.
  // The swizzles XOR bit fields that nothing else in the address uses, so
  // the address of step ks (dt) is that of step 0 with 64 ks (32 dt) XORed in.
  int kaddr[D / 32];
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) kaddr[ks] = gi * (2 * D) + 16 * ((4 * ks + G) ^ C::kswz(gi));
  const int vrow = 4 * G + gi / 4;
  const int vaddr0 = vrow * (2 * D) + 16 * (((4 * (gi % 4)) / 8) ^ C::vswz(vrow)) + 2 * ((4 * (gi % 4)) % 8);
  auto vaddr = [&](int dt) { return vaddr0 ^ (32 * dt); };

  typedef f32x4 OTiles[D / 16][2];  // O^T tile (dt, qt)
  auto zero_o = [](OTiles& o) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int i = 0; i < 4; ++i) o[dt][qt][i] = 0.0f;
  };
  OTiles oacc;
  zero_o(oacc);
  float m_run[2] = {0.0f, 0.0f};
  float l_run[2] = {0.0f, 0.0f};
  bool first = true;
  const float sl2 = p.scale_log2;

  // Sweep start.  Workgroups resident per XCD: 32 CUs x 4 SIMDs x kWaves /
  // 2 waves each.  A workgroup walks its whole list (all nk blocks of the
  // circle) in one lifetime T, so the XCD's resident workgroups share L2
  // tiles when each starts where the sweep front is at its start time: the
  // front is at 0 at launch and back at 0 after every lifetime.  Launch
  // slot (generation g, index i) starts at about g T + s_g T (i / R - 1/2):
  // the first generation starts together (s_0 = 0), and each later one
  // spreads its starts over a wider window as the finishing times drift
  // apart, s_g = min(1, 0.7 sqrt(g)) (fitted to measured start times).
  // The start is a function of the launch slot only, so the walk order --
  // and the result's bits -- do not depend on timing.
  constexpr int kResident = 64 * HalfOccupancy<D>::kWaves;
  const int slot0 = blockIdx.x / kNumXcd;
  int n0;
  {
    const int gen = slot0 / kResident, i = slot0 - gen * kResident;
    const float spread = fminf(1.0f, 0.7f * sqrtf((float)gen));
    const float front = spread * (((float)i + 0.5f) / (float)kResident - 0.5f);
    n0 = (int)floorf(front * (float)p.nk) % p.nk;
    if (n0 < 0) n0 += p.nk;
  }
  const int j0 = list.count_below(n0, p.gk);
  const bool one_chunk = p.top_k <= 64;
  const int r0 = j0 & 63;
  uint64_t rem0 = 0;
  if (one_chunk) {
    const uint64_t v = list.valid;
    rem0 = r0 == 0 ? v : (v >> r0) | (v << (64 - r0));
  }
  uint64_t rem = rem0;
  auto next_rot = [&](int j) -> int {
    if (one_chunk) {
      if (rem == 0) return p.top_k;
      const int bb = (int)__builtin_ctzll(rem);
      rem &= rem - 1;
      return (bb + r0) & 63;
    }
    if (j < 0 || j >= j0) {
      const int r = list.next(j < 0 ? j0 : j + 1, p.gk);
      if (r < p.top_k) return r;
      j = -1;
    }
    const int r = list.next(j + 1, p.gk);
    return r < j0 ? r : p.top_k;
  };

#pragma unroll
  for (int qt = 0; qt < 2; ++qt)
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) asm volatile("" ::"v"(qf[qt][ks]));

  vec8 pf[2];  // P^T of the current half, per query tile
  f32x4 sacc[2][2];
  // S^T of a 32-key K half tile at Ks.
  auto qk = [&](const uint8_t* Ks) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
#pragma unroll
        for (int i = 0; i < 4; ++i) sacc[kt][qt][i] = 0.0f;
    constexpr int kReads = 2 * (D / 32);  // read r: D step r / 2, key tile r % 2
    constexpr int kPf = 3;
    vec8 kf[kReads];
    auto read_k = [&](int r) {
      kf[r] = __builtin_bit_cast(vec8,
                                 *reinterpret_cast<const u32x4*>(Ks + kaddr[r / 2] + kGroup * (r % 2)));
    };
#pragma unroll
    for (int r = 0; r < kPf; ++r) read_k(r);
    __builtin_amdgcn_sched_group_barrier(0x100, kPf, 0);
#pragma unroll
    for (int r = 0; r < kReads; ++r) {
      if (r + kPf < kReads) read_k(r + kPf);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt)
        sacc[r % 2][qt] = Mfma<T>::mma(kf[r], qf[qt][r / 2], sacc[r % 2][qt]);
      if (r + kPf < kReads) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
  };
  // Row max of query tile qt over the half (all four lane groups), unscaled.
  auto rowmax = [&](int qt) {
    float mx = fmax3(sacc[0][qt][0], sacc[0][qt][1], sacc[0][qt][2]);
    mx = fmax3(mx, sacc[0][qt][3], sacc[1][qt][0]);
    mx = fmax3(mx, sacc[1][qt][1], sacc[1][qt][2]);
    mx = fmax3(mx, sacc[1][qt][3], sacc[1][qt][3]);
    return max_quarters(mx);
  };
  // P of query tile qt against the offset m_run[qt]; returns the sum of its
  // 8 (rounded) values.
  auto exps = [&](int qt) {
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pf[qt][4 * kt + i] = from_f32<T>(fast_exp2(fmaf(sacc[kt][qt][i], sl2, -m_run[qt])));
    return Mfma<T>::sum8(pf[qt], 0.0f);
  };
  // O^T += V^T P^T over a 32-key V half tile at Vs.
  auto pv = [&](const uint8_t* Vs, OTiles& o) {
    constexpr int kDt = D / 16;
    constexpr int kPf = 2;
    vec8 vf[kDt];
    auto read_v = [&](int dt) {
      const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(Vs + vaddr(dt)));
      const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(Vs + vaddr(dt) + kGroup));
      vf[dt] = __builtin_bit_cast(vec8, (short __attribute__((ext_vector_type(8)))){
                                            lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
    };
#pragma unroll
    for (int dt = 0; dt < kPf; ++dt) read_v(dt);
    __builtin_amdgcn_sched_group_barrier(0x100, 2 * kPf, 0);
#pragma unroll
    for (int dt = 0; dt < kDt; ++dt) {
      if (dt + kPf < kDt) read_v(dt + kPf);
#pragma unroll
      for (int qt = 0; qt < 2; ++qt) o[dt][qt] = Mfma<T>::mma(vf[dt], pf[qt], o[dt][qt]);
      if (dt + kPf < kDt) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
  };

  // Overflow guard.  A wave whose half-tile P sum passes kMaxTileSum (its
  // offset, set by the first half, is too low for a later key) marks itself
  // dirty and walks on.  If either wave of the workgroup is dirty, both find
  // each row's exact maximum over all listed keys and walk again with it as
  // the offset (every P <= 1).  Rescaling O inside the walk instead would
  // cost the walk its register allocation.
  __shared__ int wave_dirty[2];
  bool redo = false;
  for (;;) {
    zero_o(oacc);
    l_run[0] = l_run[1] = 0.0f;
    first = !redo;
    bool dirty = false;
    rem = rem0;
    int j = next_rot(-1);
    int32_t tok = j < p.top_k ? list.token(j) : 0;
    if (j < p.top_k) {
      dma(tok, 0, 0, 0);
      dma(tok, 0, 1, 1);
    }
    auto run_block = [&](auto phase) {
      constexpr int PH = decltype(phase)::value;
      const int jn = next_rot(j);
      const bool more = jn < p.top_k;
      const int32_t tokn = more ? list.token(jn) : 0;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        // ===== K half: S^T = K Q^T, then P.
        wait_vmcnt<kLoads>();
        __syncthreads();
        {
          const int t = 2 * half;
          if (half == 0) dma(tok, 1, 0, (PH + t + 2) % 3);
          else if (more) dma(tokn, 0, 0, (PH + t + 2) % 3);
        }
        qk(ring + ((PH + 2 * half) % 3) * kSlotBytes);
        if (first) {
          m_run[0] = rowmax(0) * sl2;
          m_run[1] = rowmax(1) * sl2;
        }
        const float l0 = exps(0), l1 = exps(1);
        if (__ballot(!(l0 + l1 <= kMaxTileSum))) dirty = true;  // wave-uniform, rare
        l_run[0] += l0;
        l_run[1] += l1;
        first = false;

        // ===== V half: O^T += V^T P^T over its 32 keys.
        if (half == 1 && !more)
          wait_vmcnt<0>();
        else
          wait_vmcnt<kLoads>();
        __syncthreads();
        {
          const int t = 2 * half + 1;
          if (half == 0) dma(tok, 1, 1, (PH + t + 2) % 3);
          else if (more) dma(tokn, 0, 1, (PH + t + 2) % 3);
        }
        pv(ring + ((PH + 2 * half + 1) % 3) * kSlotBytes, oacc);
      }
      j = jn;
      tok = tokn;
    };
    while (j < p.top_k) {
      run_block(Phase<0>{});
      if (j >= p.top_k) break;
      run_block(Phase<1>{});
      if (j >= p.top_k) break;
      run_block(Phase<2>{});
    }
    if (lane == 0) wave_dirty[wave] = dirty ? 1 : 0;
    __syncthreads();  // every ring read done (no DMA is outstanding here); flags visible
    if (redo || !(wave_dirty[0] | wave_dirty[1])) break;  // workgroup-uniform
    // Exact row maxima: K half tiles through slot 0, one at a time.
    float mx0 = -__builtin_inff(), mx1 = -__builtin_inff();
    for (int jj = list.next(0, p.gk); jj < p.top_k; jj = list.next(jj + 1, p.gk)) {
      const int32_t tk = list.token(jj);
      for (int half = 0; half < 2; ++half) {
        dma(tk, half, 0, 0);
        wait_vmcnt<0>();
        __syncthreads();  // both waves' rows landed
        qk(ring);
        mx0 = fmax3(mx0, rowmax(0), mx0);
        mx1 = fmax3(mx1, rowmax(1), mx1);
        __syncthreads();  // slot 0 read by both waves before it is loaded again
      }
    }
    m_run[0] = mx0 * sl2;
    m_run[1] = mx1 * sl2;
    redo = true;
  }

  // ---- Normalise and stage the 64 x D output tile in the ring (wave w's
  // rows in bytes [8 KB w, 8 KB (w + 1))), then write whole rows.
#pragma unroll
  for (int qt = 0; qt < 2; ++qt) {
    const float l_tot = sum_quarters(l_run[qt]);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    const int row = 32 * wave + 16 * qt + gi;
    uint8_t* orow = ring + row * (2 * D);
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      u32x2 w;
      w[0] = bits16(from_f32<T>(oacc[dt][qt][0] * inv)) | (bits16(from_f32<T>(oacc[dt][qt][1] * inv)) << 16);
      w[1] = bits16(from_f32<T>(oacc[dt][qt][2] * inv)) | (bits16(from_f32<T>(oacc[dt][qt][3] * inv)) << 16);
      const int chunk = 2 * dt + G / 2;  // D 16 dt + 4 G .. + 3
      *reinterpret_cast<u32x2*>(orow + 16 * (chunk ^ C::kswz(row)) + 8 * (G % 2)) = w;
    }
  }
  __syncthreads();
  {
    const int32_t tok0 = block_base_token(p.g, qb);
#pragma unroll
    for (int u = 0; u < 64 * C::DC / C::kThreads; ++u) {
      const int pidx = tid + C::kThreads * u;
      const int row = pidx / C::DC;
      const int c = pidx % C::DC;
      const int32_t t = tok0 + voxel_row_offset(p.g, row);
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(ring + row * (2 * D) + 16 * (c ^ C::kswz(row))),
                                  reinterpret_cast<u32x4*>(obase + (int64_t)t * p.o_ss + 8 * c));
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
  const int qb = p.order ? uniform_i32(p.order[wid]) : wid - bh * p.nb;
  if ((uint32_t)qb >= (uint32_t)p.nb) return;  // a launch-order entry outside [0, nb): nothing to do
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

  for (int j = next_valid(list, 0, p.top_k, p.nk); j < p.top_k;
       j = next_valid(list, j + 1, p.top_k, p.nk)) {
    const int32_t tok0 = block_base_token(p.gk, uniform_i32(list[j]));
    for (int half = 0; half < 64; half += KH) {
      __syncthreads();
      for (int i = tid; i < KH * D; i += 256) {
        const int kr = i / D;
        const int d = i - kr * D;
        const int32_t tok = tok0 + voxel_row_offset(p.gk, half + kr);
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
  hipLaunchKernelGGL((attn_half_kernel<T, D>), dim3(grid), dim3(128), 0, stream, p);
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
  // Every dtype has the vector-ALU kernel at these head dims.
  const bool dtype_ok = dtype == LCV_BSA_F16 || dtype == LCV_BSA_BF16 || dtype == LCV_BSA_F32;
  return dtype_ok && (D == 16 || D == 32 || D == 64 || D == 128 || D == 256);
}

hipError_t launch_attn(const AttnParams& p, int dtype, int D, hipStream_t stream) {
  if (attn_uses_mfma(dtype, D) && p.scale_log2 >= 0.0f) {
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
