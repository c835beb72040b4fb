/*
 * lcv_bsa.h -- C ABI of the MI355X (gfx950) Block Sparse Attention forward.
 *
 * Every pointer argument is a DEVICE pointer unless stated otherwise.
 * Dimensions are int64_t; strides are in ELEMENTS (not bytes) and the head
 * dimension (last axis) must have stride 1.  `stream` is a hipStream_t passed
 * as void* (NULL = the null stream).  Nothing here allocates or frees memory,
 * synchronises the device, or retains a pointer past the call: outputs and
 * workspaces are owned by the caller.  All launches are stream ordered.
 *
 * Tensor conventions follow the reference (longcat_video/models/
 * block_sparse_attention.py): q, k, v are [B, H, S, D] with S = T*Hl*Wl
 * flattened t-major over the latent grid (T, Hl, Wl).  A block is a
 * cT x cH x cW voxel of that grid; blocks are numbered bt*Bh*Bw + bh*Bw + bw
 * (Bt = T/cT, Bh = Hl/cH, Bw = Wl/cW) and the rows inside a block are ordered
 * (i, j, l) row-major over the voxel (the reference's block-major order).
 * Contiguous 64-token blocks are the grid (1, 1, S) with chunk (1, 1, 64).
 *
 * Return value: LCV_BSA_OK (0) or one of the LCV_BSA_ERR_* codes; the
 * calling thread's last error text is available from lcv_bsa_last_error().
 */
#ifndef LCV_BSA_H
#define LCV_BSA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types of q / k / v / out. */
enum lcv_bsa_dtype {
  LCV_BSA_F16 = 0,
  LCV_BSA_BF16 = 1,
  LCV_BSA_F32 = 2
};

/* Status codes. */
enum lcv_bsa_status {
  LCV_BSA_OK = 0,
  LCV_BSA_ERR_INVALID_ARG = 1,  /* null pointer, non-positive dimension   */
  LCV_BSA_ERR_SHAPE = 2,        /* S != T*Hl*Wl, grid not a chunk multiple */
  LCV_BSA_ERR_DTYPE = 3,        /* unknown dtype enum                       */
  LCV_BSA_ERR_UNSUPPORTED = 4,  /* valid but unsupported (D, block size)    */
  LCV_BSA_ERR_LAYOUT = 5,       /* stride / alignment the kernels can't use */
  LCV_BSA_ERR_LAUNCH = 6        /* HIP runtime error at launch              */
};

/* Geometry of the latent grid and of one block (voxel). */
typedef struct lcv_bsa_geom {
  int64_t T, Hl, Wl;  /* latent grid; S must equal T*Hl*Wl   */
  int64_t cT, cH, cW; /* voxel; each must divide its grid axis */
} lcv_bsa_geom;

/* Strides (in elements) of a [B, H, S, D] tensor whose D axis is dense. */
typedef struct lcv_bsa_strides {
  int64_t b, h, s;
} lcv_bsa_strides;

/* Library version string, e.g. "lcv_bsa 0.1.0 gfx950". Host only. */
const char* lcv_bsa_version(void);

/* Static text for a status code. Host only. */
const char* lcv_bsa_strerror(int status);

/* Detailed text of the calling thread's most recent failure ("" if none). */
const char* lcv_bsa_last_error(void);

/*
 * Block-mean pooling.  out[b,h,n,:] = mean of the cT*cH*cW rows of block n,
 * accumulated in fp32.  out is a dense [B, H, nb, D] fp32 tensor,
 * nb = (T/cT)*(Hl/cH)*(Wl/cW).
 * Replaces mean_pool_blocks_3d, longcat_video/models/block_sparse_attention.py:67-104
 * (called from longcat_video/models/attention.py:103-104).
 */
int lcv_bsa_pool(const void* x, int dtype, int64_t B, int64_t H, int64_t S,
                 int64_t D, lcv_bsa_strides xs, lcv_bsa_geom g, float* out,
                 void* stream);

/*
 * Block routing scores: score[b,h,i,j] = dot(qbar[b,h,i,:], kbar[b,h,j,:])
 * in fp32, unscaled.  qbar [B,H,nq,D], kbar [B,H,nk,D], score [B,H,nq,nk],
 * all dense fp32.  D % 4 == 0, D <= 256.
 * Replaces block_routing_scores, block_sparse_attention.py:107-112.
 */
int lcv_bsa_scores(const float* qbar, const float* kbar, int64_t B, int64_t H,
                   int64_t nq, int64_t nk, int64_t D, float* score,
                   void* stream);

/*
 * Per-row top-k of a dense fp32 score tensor [B,H,nq,nk] -> idx [B,H,nq,top_k]
 * int32.  Each row's set is the top_k largest scores; among equal scores
 * the lower block index wins; NaN ranks below -inf; -0.0 equals +0.0.
 * Indices are written in ascending order.  1 <= top_k <= nk <= 4096.
 * Replaces topk_block_indices, block_sparse_attention.py:115-134
 * (the reference returns the same set in unspecified order).
 */
int lcv_bsa_topk(const float* score, int64_t B, int64_t H, int64_t nq,
                 int64_t nk, int64_t top_k, int32_t* idx, void* stream);

/*
 * Fused routing: scores of qbar x kbar^T kept on chip, then the per-row
 * top-k of lcv_bsa_topk.  Same arguments and result as lcv_bsa_scores
 * followed by lcv_bsa_topk, without the [B,H,nq,nk] intermediate.
 * Replaces block_sparse_attention.py:230-233 (attention.py:105-108).
 */
int lcv_bsa_select(const float* qbar, const float* kbar, int64_t B, int64_t H,
                   int64_t nq, int64_t nk, int64_t D, int64_t top_k,
                   int32_t* idx, void* stream);

/*
 * Launch order for lcv_bsa_attn_fwd: per (b,h), a permutation of the nq
 * q-blocks sorted by (first, middle) entry of their routing lists, so that
 * q-blocks whose ascending lists start together run together and share K/V
 * tiles in L2.  order is a dense [B,H,nq] int32.  Any permutation gives the
 * same attention result up to fp32 rounding (each workgroup starts its
 * ascending list at an entry set by its launch slot, which changes the
 * summation order); for a given order the result is deterministic.
 * nq <= 4096.
 * No counterpart in the reference (its kernels launch in block order).
 */
int lcv_bsa_schedule(const int32_t* idx, int64_t B, int64_t H, int64_t nq,
                     int64_t top_k, int32_t* order, void* stream);

/*
 * lcv_bsa_schedule for routing lists over nk K/V blocks (S_q != S_k, the
 * input of lcv_bsa_attn_fwd_kv): list entries are K/V block ids in [0, nk)
 * and sort by their value up to nk (lcv_bsa_schedule is this with nk = nq).
 * nq <= 4096, nk < 2^20.  No counterpart in the reference, whose layer sends
 * S_q != S_k to dense attention (attention.py:89, 218-221, 273).
 */
int lcv_bsa_schedule_kv(const int32_t* idx, int64_t B, int64_t H, int64_t nq,
                        int64_t nk, int64_t top_k, int32_t* order, void* stream);

/*
 * Sparse attention over given block lists (the kernel-level entry):
 *   out[b,h,s,:] = softmax_j(sm_scale * q[s].k[j]) v[j]
 * over every key j in the blocks idx[b,h,block_of(s),0..top_k-1].
 * Entries < 0 or >= nb are skipped (padding); a row with no valid block
 * gets zeros.  Duplicate entries are attended once per occurrence (the
 * reference kernels' behaviour).  idx is a dense [B,H,nb,top_k] int32.
 * order (nullable) is a per-head permutation of the q-blocks giving the
 * launch order (lcv_bsa_schedule); null launches in block order.  An order
 * entry outside [0, nb) launches nothing (that slot's work is skipped, so a
 * non-permutation leaves some output rows unwritten).
 * Blocks must hold 64 tokens.  D in {16,32,64,128,256} (MFMA path for
 * fp16/bf16 with D in {64,128}; other combinations use a vector-ALU path).
 * Replaces bsa_attention_metal_v4 / _v3 / _v2 / bsa_attention_metal,
 * longcat_video/models/block_sparse_attention_metal.py:985-1046 (and
 * 729-810, 484-548, 224-295): their block-major reshapes (185-221) are
 * folded into the kernel's row addressing.
 */
int lcv_bsa_attn_fwd(const void* q, const void* k, const void* v, int dtype,
                     int64_t B, int64_t H, int64_t S, int64_t D,
                     lcv_bsa_strides qs, lcv_bsa_strides ks,
                     lcv_bsa_strides vs, const int32_t* idx,
                     const int32_t* order, int64_t top_k, float sm_scale,
                     lcv_bsa_geom g, void* out, lcv_bsa_strides os,
                     void* stream);

/*
 * lcv_bsa_attn_fwd with q and k / v of different lengths and block
 * geometries: q and out have Sq rows cut by gq into nq 64-token blocks, k
 * and v have Sk rows cut by gk into nk blocks; idx is a dense
 * [B,H,nq,top_k] int32 of k/v block ids (entries outside [0, nk) are
 * skipped) and order a per-head permutation of the nq q-blocks (nullable).
 * This is BSA for the conditioning / KV-cache paths of the reference, where
 * noise queries attend to cached + new keys
 * (longcat_video/models/attention.py:218-221 and 235-275), which the
 * reference always sends to dense attention (attention.py:89 requires
 * S_q == S_k).  With Sq == Sk and gq == gk it is lcv_bsa_attn_fwd.
 */
int lcv_bsa_attn_fwd_kv(const void* q, const void* k, const void* v, int dtype,
                        int64_t B, int64_t H, int64_t Sq, int64_t Sk, int64_t D,
                        lcv_bsa_strides qs, lcv_bsa_strides ks,
                        lcv_bsa_strides vs, const int32_t* idx,
                        const int32_t* order, int64_t top_k, float sm_scale,
                        lcv_bsa_geom gq, lcv_bsa_geom gk, void* out,
                        lcv_bsa_strides os, void* stream);

/*
 * DiT block row operation (one pass over [B, N, C] rows, fp16 / bf16):
 *   r = x                      (a null)
 *     = round(x + a)           (a given, gate null)
 *     = round(x + gate * a)    (gate: fp32 [B, frames, C], per latent frame)
 * written to x_out when given; then, when n_out is given,
 *   y = LayerNorm_fp32(r; eps)  [* ln_weight + ln_bias]  [* (scale + 1) + shift]
 * rounded to the dtype (shift / scale: fp32 [B, frames, C]).  N must be a
 * multiple of frames (tokens of frame t: rows t*N/frames ..); C % 8 == 0,
 * C <= 8192; every pointer 16-byte aligned, tensors contiguous.
 * Replaces, in LongCatSingleStreamBlock.__call__ (longcat_video/models/
 * longcat_video_dit.py:107-136): modulate_fp32 over LayerNorm_FP32
 * (blocks.py:79-119), the fp32 gated residuals, the cross-attention residual
 * and pre_crs_attn_norm -- each a chain of full-tensor passes there.
 */
int lcv_bsa_block_rows(const void* x, const void* a, int dtype, int64_t B,
                       int64_t N, int64_t C, int64_t frames, const float* gate,
                       const float* shift, const float* scale,
                       const void* ln_weight, const void* ln_bias, float eps,
                       void* x_out, void* n_out, void* stream);

/*
 * SwiGLU gate: out[r, j] = round(round(silu(h[r, j])) * h[r, hidden + j])
 * for h = [rows, 2*hidden] (the w1 and w3 projections side by side) and
 * out = [rows, hidden].  fp16 / bf16, hidden % 8 == 0, 16-byte aligned.
 * Replaces silu(w1(x)) * w3(x) of FeedForwardSwiGLU (blocks.py:50-51).
 */
int lcv_bsa_block_swiglu(const void* h13, int dtype, int64_t rows,
                         int64_t hidden, void* out, void* stream);

/*
 * Per-head RMSNorm_FP32 (blocks.py:55-72) of a [B,H,S,D] view into another
 * [B,H,S,D] view (strides in elements, any layout with dense D):
 *   out = round(round(x * rsqrt(mean(x^2) + eps)) * weight).
 * weight: [D] in the dtype, or null for 1.  D in {64, 128}.  Used for the
 * cross-attention's q_norm / k_norm (attention.py:325-326), reading the
 * projection's [B, S, H, D] rows and writing the layout attention reads.
 */
int lcv_bsa_head_rms_norm(const void* x, int dtype, int64_t B, int64_t H,
                          int64_t S, int64_t D, lcv_bsa_strides xs,
                          const void* weight, float eps, void* out,
                          lcv_bsa_strides os, void* stream);

/*
 * Bytes of workspace lcv_bsa_forward needs: the fp32 pooled means of q and
 * k (2*B*H*nb*D*4 bytes), the fp32 block scores (B*H*nb*nb*4 bytes) and the
 * int32 launch order (B*H*nb*4 bytes), each rounded up to 256 bytes.  Host
 * only.
 */
size_t lcv_bsa_forward_workspace_bytes(int64_t B, int64_t H, int64_t nb,
                                       int64_t D);

/*
 * End-to-end block sparse attention: pool q and k, route (scores + top-k),
 * schedule, then sparse attention.  idx receives the [B,H,nb,top_k] routing
 * (ascending per row); workspace holds at least
 * lcv_bsa_forward_workspace_bytes() bytes, 256-byte aligned.
 * Replaces bsa_attention, block_sparse_attention.py:201-250, whose result
 * equals this one (its masked entries contribute exactly zero).
 */
int lcv_bsa_forward(const void* q, const void* k, const void* v, int dtype,
                    int64_t B, int64_t H, int64_t S, int64_t D,
                    lcv_bsa_strides qs, lcv_bsa_strides ks,
                    lcv_bsa_strides vs, int64_t top_k, float sm_scale,
                    lcv_bsa_geom g, void* workspace, size_t workspace_bytes,
                    int32_t* idx, void* out, lcv_bsa_strides os,
                    void* stream);

/* Bytes of device scratch lcv_bsa_forward_noalloc holds per GPU. */
#define LCV_BSA_NOALLOC_SCRATCH_BYTES ((size_t)1 << 20)

/*
 * lcv_bsa_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  No counterpart in the
 * reference.  Same arguments and result as lcv_bsa_forward.  The call
 * allocates and frees nothing:
 *   - the launch order (one int32 per (b, h, q-block)) lives in a fixed
 *     device array of LCV_BSA_NOALLOC_SCRATCH_BYTES that every GPU the
 *     library runs on holds until the process ends:
 *     round256(B*H*nb*4) <= 1 MiB, i.e. B*H*nb <= 262,144 (720p at H=32,
 *     nb=900: 28,800); larger problems get LCV_BSA_ERR_UNSUPPORTED before
 *     any device work;
 *   - the pooled means of q and k and the block scores are staged in out
 *     before the attention overwrites every element of it.  out must
 *     therefore be dense (its B*H*S*D elements fill one range, in any
 *     order of the b, h, s dimensions; else LCV_BSA_ERR_LAYOUT) and must
 *     overlap none of q, k, v, idx (else LCV_BSA_ERR_INVALID_ARG).
 * out holds 64*D elements per block, the means 2*D floats, so the means
 * always fit; the rest holds the block scores of as many (b, h) pairs as
 * fit (every head at 720p), and the routing runs as score GEMM + top-k over
 * those slices when at most 8 slices cover every head, else as the fused
 * select kernel that keeps the scores on chip (with a 2-byte out, when
 * num_blocks is above about 30*B*H*D or 240*D).  At D = 64 or 128 with num_blocks <= 2048 the fused
 * kernel computes every score with the same split-bf16 MFMA sequence as
 * the score GEMM, so both routes select the same blocks; elsewhere the
 * fused kernel sums in fp32 on the vector ALU, and two scores within fp32
 * rounding of each other may then be ordered differently than
 * lcv_bsa_forward orders them.
 * The first call on each device resolves the array's device address and
 * creates an event; it must not be under stream capture (it returns
 * LCV_BSA_ERR_UNSUPPORTED there, before any device work); later calls may
 * be captured.  Calls on one GPU share its array.  Uncaptured calls are
 * ordered by the library: one on another stream than the previous
 * uncaptured call waits (hipStreamWaitEvent) for that call's work, and
 * calls from several host threads queue on a lock.  Captured calls are not:
 * a graph replay that overlaps in time with another call on the same GPU
 * races on the launch order, and the caller must order the two.  Nothing in
 * the array carries over from one call to the next (each call writes every
 * byte it reads).
 */
int lcv_bsa_forward_noalloc(const void* q, const void* k, const void* v,
                            int dtype, int64_t B, int64_t H, int64_t S,
                            int64_t D, lcv_bsa_strides qs, lcv_bsa_strides ks,
                            lcv_bsa_strides vs, int64_t top_k, float sm_scale,
                            lcv_bsa_geom g, int32_t* idx, void* out,
                            lcv_bsa_strides os, void* stream);

/*
 * Token -> block map: out[s] = block of token s (int32, length T*Hl*Wl).
 * Replaces build_token_block_indices, block_sparse_attention.py:137-159.
 */
int lcv_bsa_token_blocks(lcv_bsa_geom g, int32_t* out, void* stream);

/*
 * Token-pair mask: mask[b,h,sq,sk] = 1 if token_block[sk] is listed in
 * idx[b,h,token_block[sq],:], else 0 (uint8, dense [B,H,S,S]).
 * idx is a dense [B,H,nq,top_k] int32 routing, token_block a length-S int32
 * map into [0, nq) (as lcv_bsa_token_blocks writes); num_kv_blocks bounds the
 * listed entries (those outside [0, num_kv_blocks) match nothing).  Only
 * sensible for small S (B*H*S*S <= 2^34).
 * Replaces build_token_pair_mask, block_sparse_attention.py:162-198.
 */
int lcv_bsa_token_pair_mask(const int32_t* idx, int64_t B, int64_t H,
                            int64_t nq, int64_t top_k,
                            const int32_t* token_block, int64_t S,
                            int64_t num_kv_blocks, uint8_t* mask,
                            void* stream);

/*
 * t-major <-> block-major row permutation of a [B,H,S,D] tensor (dense in
 * and out, same dtype).  inverse = 0: out row (block n, row r) = x row of
 * that token; inverse = 1: the reverse.
 * Replaces _reshape_to_block_major / _reshape_from_block_major,
 * block_sparse_attention_metal.py:185-221.
 */
int lcv_bsa_permute_block_major(const void* x, int dtype, int64_t B,
                                int64_t H, int64_t S, int64_t D,
                                lcv_bsa_geom g, int inverse, void* out,
                                void* stream);

/*
 * Latent grid of the 3D RoPE (t-major token order): S = T * Hl * Wl.
 */
typedef struct lcv_bsa_grid {
  int64_t T, Hl, Wl;
} lcv_bsa_grid;

/*
 * Length (floats) of the RoPE table lcv_bsa_prepare_qk reads, for head dim D
 * split into t / h / w parts of dt = D - 4*(D/6), dh = dw = 2*(D/6) dims
 * (longcat_video/models/rope_3d.py:60-62).  Layout, each part row-major over
 * [position][pair]:
 *   cos_t[T][dt/2], sin_t[T][dt/2], cos_h[Hl][dh/2], sin_h[Hl][dh/2],
 *   cos_w[Wl][dw/2], sin_w[Wl][dw/2]
 * with angle(axis position p, pair i) = p / 10000^(2i / dim_axis)
 * (rope_3d.py:65-93).  Returns 0 when D or the grid is not supported
 * (D in {64, 128}, length <= 12288).
 */
int64_t lcv_bsa_rope_table_len(int64_t D, lcv_bsa_grid rope);

/*
 * Pre-BSA preparation of q and k in one pass (no reference counterpart as a
 * single function; replaces the q_norm / k_norm / rope_3d steps of
 * Attention.__call__, longcat_video/models/attention.py:195-201, plus
 * mean_pool_blocks_3d, block_sparse_attention.py:67-104):
 *   q_out = rope_3d(RMSNorm_FP32(q_in)), k_out likewise, where RMSNorm_FP32
 *   (longcat_video/models/blocks.py:55-72) is x * rsqrt(mean(x^2) + eps) in
 *   fp32, rounded to the dtype, times the weight (dtype [D]; NULL = ones),
 *   and rope_3d (rope_3d.py:107-128) rotates in fp32 and rounds back;
 *   qbar / kbar = fp32 block means of q_out / k_out ([B,H,nb,D], as
 *   lcv_bsa_pool).
 * fp16/bf16 only; D in {64, 128}; 64-token blocks (geometry g); rope is the
 * latent grid of the RoPE positions (its product must be S); rope_table as
 * described at lcv_bsa_rope_table_len.  All tensors 16-byte aligned rows.
 */
int lcv_bsa_prepare_qk(const void* q_in, const void* k_in, int dtype,
                       int64_t B, int64_t H, int64_t S, int64_t D,
                       lcv_bsa_strides q_in_strides, lcv_bsa_strides k_in_strides,
                       const void* q_weight, const void* k_weight, float eps,
                       lcv_bsa_grid rope, const float* rope_table,
                       int64_t rope_table_len, lcv_bsa_geom g,
                       void* q_out, void* k_out, lcv_bsa_strides q_out_strides,
                       lcv_bsa_strides k_out_strides, float* qbar, float* kbar,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LCV_BSA_H */
