// C ABI entry points: argument validation, geometry checks and launches.
//
// The shape contract mirrors the reference's ValueError checks
// (longcat_video/models/block_sparse_attention.py:86-96 and
// longcat_video/models/block_sparse_attention_metal.py:257-262, 1003-1017):
// a violation returns LCV_BSA_ERR_SHAPE / _UNSUPPORTED with the reason in
// lcv_bsa_last_error(), which the Python layer turns into ValueError.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <cmath>
#include <mutex>

#include "bsa_common.h"

#define LCV_BSA_VERSION "lcv_bsa 0.1.0 gfx950"

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return status;
}

int ok() {
  g_last_error[0] = '\0';
  return LCV_BSA_OK;
}

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess)
    return fail(LCV_BSA_ERR_LAUNCH, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
  return ok();
}

bool dtype_ok(int dtype) {
  return dtype == LCV_BSA_F16 || dtype == LCV_BSA_BF16 || dtype == LCV_BSA_F32;
}

int elem_bytes(int dtype) { return dtype == LCV_BSA_F32 ? 4 : 2; }

constexpr int64_t kI32Max = 2147483647;

// Validates (B, H, S, D) and the grid/voxel geometry; fills nb and bs.
int check_geom(int64_t B, int64_t H, int64_t S, int64_t D, const lcv_bsa_geom& g, int64_t* nb,
               int64_t* bs) {
  if (B <= 0 || H <= 0 || S <= 0 || D <= 0)
    return fail(LCV_BSA_ERR_INVALID_ARG, "B, H, S, D must be positive (got %lld, %lld, %lld, %lld)",
                (long long)B, (long long)H, (long long)S, (long long)D);
  if (g.T <= 0 || g.Hl <= 0 || g.Wl <= 0 || g.cT <= 0 || g.cH <= 0 || g.cW <= 0)
    return fail(LCV_BSA_ERR_INVALID_ARG, "grid and chunk extents must be positive");
  // Bound every factor before the products below (no int64 overflow).
  if (S > kI32Max / 2 || B > kI32Max || H > kI32Max || D > kI32Max || g.T > kI32Max ||
      g.Hl > kI32Max || g.Wl > kI32Max || g.cT > kI32Max || g.cH > kI32Max || g.cW > kI32Max)
    return fail(LCV_BSA_ERR_UNSUPPORTED, "S=%lld or an extent beyond 2^31", (long long)S);
  if (g.T % g.cT || g.Hl % g.cH || g.Wl % g.cW)
    return fail(LCV_BSA_ERR_SHAPE,
                "Latent shape (%lld, %lld, %lld) must be a multiple of chunk_thw (%lld, %lld, %lld)",
                (long long)g.T, (long long)g.Hl, (long long)g.Wl, (long long)g.cT, (long long)g.cH,
                (long long)g.cW);
  const int64_t thw = g.T * g.Hl > S ? -1 : g.T * g.Hl * g.Wl;  // factors < 2^31: no overflow
  if (S != thw)
    return fail(LCV_BSA_ERR_SHAPE, "S=%lld doesn't match T*H*W=%lld*%lld*%lld", (long long)S,
                (long long)g.T, (long long)g.Hl, (long long)g.Wl);
  if (B * H > kI32Max / 4)
    return fail(LCV_BSA_ERR_UNSUPPORTED, "B*H=%lld too large", (long long)(B * H));
  *bs = g.cT * g.cH * g.cW;
  *nb = S / *bs;
  if (B * H * (*nb) > kI32Max)
    return fail(LCV_BSA_ERR_UNSUPPORTED, "B*H*num_blocks too large");
  return LCV_BSA_OK;
}

int check_strides(const char* name, const lcv_bsa_strides& s, int64_t D) {
  if (s.b < 0 || s.h < 0 || s.s < D)
    return fail(LCV_BSA_ERR_LAYOUT,
                "%s strides (b=%lld, h=%lld, s=%lld) must be non-negative with s >= D=%lld "
                "(the head dimension must be dense)",
                name, (long long)s.b, (long long)s.h, (long long)s.s, (long long)D);
  return LCV_BSA_OK;
}

bool vec_aligned(const void* p, const lcv_bsa_strides& s, int vec) {
  return ((uintptr_t)p & 15u) == 0 && s.b % vec == 0 && s.h % vec == 0 && s.s % vec == 0;
}

// Bytes from the first to one past the last element of one head.
uint64_t head_bytes(int64_t S, int64_t row_stride, int64_t D, int dtype) {
  return (uint64_t)((S - 1) * row_stride + D) * (uint64_t)elem_bytes(dtype);
}

// q / out have S rows in geometry g (nb blocks); k / v have Sk rows in
// geometry gk (nk blocks).
int check_attn_args(const void* q, const void* k, const void* v, const void* out, int dtype,
                    int64_t B, int64_t H, int64_t S, int64_t Sk, int64_t D,
                    const lcv_bsa_strides& qs, const lcv_bsa_strides& ks,
                    const lcv_bsa_strides& vs, const lcv_bsa_strides& os, int64_t top_k,
                    float sm_scale, const lcv_bsa_geom& g, const lcv_bsa_geom& gk, int64_t* nb,
                    int64_t* nk, int64_t* bs) {
  if (!q || !k || !v || !out) return fail(LCV_BSA_ERR_INVALID_ARG, "null tensor pointer");
  if (!dtype_ok(dtype)) return fail(LCV_BSA_ERR_DTYPE, "unknown dtype %d", dtype);
  int st = check_geom(B, H, S, D, g, nb, bs);
  if (st) return st;
  if (*bs != 64)
    return fail(LCV_BSA_ERR_UNSUPPORTED,
                "block size cT*cH*cW=%lld: the attention kernels require 64-token blocks",
                (long long)*bs);
  int64_t bsk = 0;
  if ((st = check_geom(B, H, Sk, D, gk, nk, &bsk))) return st;
  if (bsk != 64)
    return fail(LCV_BSA_ERR_UNSUPPORTED,
                "k/v block size cT*cH*cW=%lld: the attention kernels require 64-token blocks",
                (long long)bsk);
  if (!lcv::attn_supported(dtype, (int)D))
    return fail(LCV_BSA_ERR_UNSUPPORTED, "head_dim D=%lld unsupported (D in {16,32,64,128,256})",
                (long long)D);
  if (top_k < 1 || top_k > kI32Max / (*nb))
    return fail(LCV_BSA_ERR_INVALID_ARG, "top_k=%lld must be >= 1", (long long)top_k);
  if (!std::isfinite(sm_scale)) return fail(LCV_BSA_ERR_INVALID_ARG, "sm_scale must be finite");
  if ((st = check_strides("q", qs, D)) || (st = check_strides("k", ks, D)) ||
      (st = check_strides("v", vs, D)) || (st = check_strides("out", os, D)))
    return st;
  if (lcv::attn_uses_mfma(dtype, (int)D)) {
    const int vec = 16 / elem_bytes(dtype);
    if (!vec_aligned(q, qs, vec) || !vec_aligned(k, ks, vec) || !vec_aligned(v, vs, vec) ||
        !vec_aligned(out, os, vec))
      return fail(LCV_BSA_ERR_LAYOUT,
                  "q/k/v/out rows must start on 16-byte boundaries (pointers 16-byte aligned, "
                  "strides multiples of %d elements)", vec);
    if (head_bytes(Sk, ks.s, D, dtype) > 0xFFFFFFFFull || head_bytes(Sk, vs.s, D, dtype) > 0xFFFFFFFFull)
      return fail(LCV_BSA_ERR_LAYOUT, "one head of k or v spans more than 4 GiB");
  }
  return LCV_BSA_OK;
}

lcv::AttnParams make_attn_params(const void* q, const void* k, const void* v, void* out,
                                 const lcv_bsa_strides& qs, const lcv_bsa_strides& ks,
                                 const lcv_bsa_strides& vs, const lcv_bsa_strides& os,
                                 const int32_t* idx, const int32_t* order, int64_t B, int64_t H,
                                 int64_t Sk, int64_t D, int dtype, int64_t nb, int64_t nk,
                                 int64_t top_k, float sm_scale, const lcv_bsa_geom& g,
                                 const lcv_bsa_geom& gk) {
  lcv::AttnParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.out = out;
  p.q_sb = qs.b, p.q_sh = qs.h, p.q_ss = qs.s;
  p.k_sb = ks.b, p.k_sh = ks.h, p.k_ss = ks.s;
  p.v_sb = vs.b, p.v_sh = vs.h, p.v_ss = vs.s;
  p.o_sb = os.b, p.o_sh = os.h, p.o_ss = os.s;
  p.idx = idx;
  p.order = order;
  p.B = (int32_t)B;
  p.H = (int32_t)H;
  p.nb = (int32_t)nb;
  p.nk = (int32_t)nk;
  p.top_k = (int32_t)top_k;
  p.scale_log2 = sm_scale * 1.4426950408889634f;
  const uint64_t kb = head_bytes(Sk, ks.s, D, dtype), vb = head_bytes(Sk, vs.s, D, dtype);
  p.k_head_bytes = kb > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)kb;
  p.v_head_bytes = vb > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)vb;
  p.g = lcv::make_geom(g);
  p.gk = lcv::make_geom(gk);
  return p;
}

int check_route(int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t D, bool need_d) {
  if (B <= 0 || H <= 0 || nq <= 0 || nk <= 0 || (need_d && D <= 0))
    return fail(LCV_BSA_ERR_INVALID_ARG, "B, H, nq, nk%s must be positive", need_d ? ", D" : "");
  if (B * H * nq > kI32Max || nq * nk > kI32Max)
    return fail(LCV_BSA_ERR_UNSUPPORTED, "routing problem too large");
  if (!lcv::select_supported((int)nk, need_d ? (int)D : 4))
    return fail(LCV_BSA_ERR_UNSUPPORTED,
                "routing supports nk <= 4096 and D % 4 == 0, D <= 128 (got nk=%lld, D=%lld)",
                (long long)nk, (long long)D);
  return LCV_BSA_OK;
}

}  // namespace

extern "C" {

const char* lcv_bsa_version(void) { return LCV_BSA_VERSION; }

const char* lcv_bsa_strerror(int status) {
  switch (status) {
    case LCV_BSA_OK: return "ok";
    case LCV_BSA_ERR_INVALID_ARG: return "invalid argument";
    case LCV_BSA_ERR_SHAPE: return "shape mismatch";
    case LCV_BSA_ERR_DTYPE: return "unsupported dtype";
    case LCV_BSA_ERR_UNSUPPORTED: return "unsupported configuration";
    case LCV_BSA_ERR_LAYOUT: return "unsupported memory layout";
    case LCV_BSA_ERR_LAUNCH: return "kernel launch failed";
    default: return "unknown status";
  }
}

const char* lcv_bsa_last_error(void) { return g_last_error; }

int lcv_bsa_pool(const void* x, int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                 lcv_bsa_strides xs, lcv_bsa_geom g, float* out, void* stream) {
  if (!x || !out) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  if (!dtype_ok(dtype)) return fail(LCV_BSA_ERR_DTYPE, "unknown dtype %d", dtype);
  int64_t nb = 0, bs = 0;
  int st = check_geom(B, H, S, D, g, &nb, &bs);
  if (st) return st;
  if ((st = check_strides("x", xs, D))) return st;
  const lcv::Tensor4 t{x, xs.b, xs.h, xs.s};
  float* outs[1] = {out};
  return launch_status(lcv::launch_pool(&t, 1, dtype, (int)B, (int)H, (int)D, (int)nb, (int)bs,
                                        lcv::make_geom(g), outs, (hipStream_t)stream),
                       "lcv_bsa_pool");
}

int lcv_bsa_scores(const float* qbar, const float* kbar, int64_t B, int64_t H, int64_t nq,
                   int64_t nk, int64_t D, float* score, void* stream) {
  if (!qbar || !kbar || !score) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  int st = check_route(B, H, nq, nk, D, true);
  if (st) return st;
  return launch_status(lcv::launch_scores(qbar, kbar, (int)B, (int)H, (int)nq, (int)nk, (int)D,
                                          score, (hipStream_t)stream),
                       "lcv_bsa_scores");
}

int lcv_bsa_topk(const float* score, int64_t B, int64_t H, int64_t nq, int64_t nk, int64_t top_k,
                 int32_t* idx, void* stream) {
  if (!score || !idx) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  int st = check_route(B, H, nq, nk, 0, false);
  if (st) return st;
  if (top_k < 1 || top_k > nk)
    return fail(LCV_BSA_ERR_INVALID_ARG, "top_k=%lld must be in [1, nk=%lld]", (long long)top_k,
                (long long)nk);
  return launch_status(lcv::launch_topk(score, (int)B, (int)H, (int)nq, (int)nk, (int)top_k, idx,
                                        (hipStream_t)stream),
                       "lcv_bsa_topk");
}

int lcv_bsa_select(const float* qbar, const float* kbar, int64_t B, int64_t H, int64_t nq,
                   int64_t nk, int64_t D, int64_t top_k, int32_t* idx, void* stream) {
  if (!qbar || !kbar || !idx) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  int st = check_route(B, H, nq, nk, D, true);
  if (st) return st;
  if (top_k < 1 || top_k > nk)
    return fail(LCV_BSA_ERR_INVALID_ARG, "top_k=%lld must be in [1, nk=%lld]", (long long)top_k,
                (long long)nk);
  return launch_status(lcv::launch_select(qbar, kbar, (int)B, (int)H, (int)nq, (int)nk, (int)D,
                                          (int)top_k, idx, (hipStream_t)stream),
                       "lcv_bsa_select");
}

int lcv_bsa_schedule(const int32_t* idx, int64_t B, int64_t H, int64_t nq, int64_t top_k,
                     int32_t* order, void* stream) {
  return lcv_bsa_schedule_kv(idx, B, H, nq, nq, top_k, order, stream);
}

int lcv_bsa_schedule_kv(const int32_t* idx, int64_t B, int64_t H, int64_t nq, int64_t nk,
                        int64_t top_k, int32_t* order, void* stream) {
  if (!idx || !order) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  if (B <= 0 || H <= 0 || nq <= 0 || nk <= 0 || top_k <= 0)
    return fail(LCV_BSA_ERR_INVALID_ARG, "B, H, nq, nk, top_k must be positive");
  if (!lcv::schedule_supported((int)std::min<int64_t>(nq, kI32Max),
                               (int)std::min<int64_t>(nk, kI32Max)) ||
      B * H > kI32Max || B * H * nq * top_k > ((int64_t)1 << 40))
    return fail(LCV_BSA_ERR_UNSUPPORTED,
                "scheduling supports nq <= 4096 and nk < 2^20 (got nq=%lld, nk=%lld)",
                (long long)nq, (long long)nk);
  return launch_status(lcv::launch_schedule(idx, (int)(B * H), (int)nq, (int)nk, (int)top_k, order,
                                            (hipStream_t)stream),
                       "lcv_bsa_schedule");
}

int lcv_bsa_attn_fwd(const void* q, const void* k, const void* v, int dtype, int64_t B,
                     int64_t H, int64_t S, int64_t D, lcv_bsa_strides qs, lcv_bsa_strides ks,
                     lcv_bsa_strides vs, const int32_t* idx, const int32_t* order, int64_t top_k,
                     float sm_scale, lcv_bsa_geom g, void* out, lcv_bsa_strides os,
                     void* stream) {
  return lcv_bsa_attn_fwd_kv(q, k, v, dtype, B, H, S, S, D, qs, ks, vs, idx, order, top_k, sm_scale,
                             g, g, out, os, stream);
}

int lcv_bsa_attn_fwd_kv(const void* q, const void* k, const void* v, int dtype, int64_t B,
                        int64_t H, int64_t Sq, int64_t Sk, int64_t D, lcv_bsa_strides qs,
                        lcv_bsa_strides ks, lcv_bsa_strides vs, const int32_t* idx,
                        const int32_t* order, int64_t top_k, float sm_scale, lcv_bsa_geom gq,
                        lcv_bsa_geom gk, void* out, lcv_bsa_strides os, void* stream) {
  int64_t nq = 0, nk = 0, bs = 0;
  int st = check_attn_args(q, k, v, out, dtype, B, H, Sq, Sk, D, qs, ks, vs, os, top_k, sm_scale,
                           gq, gk, &nq, &nk, &bs);
  if (st) return st;
  if (!idx) return fail(LCV_BSA_ERR_INVALID_ARG, "null block index pointer");
  const lcv::AttnParams p = make_attn_params(q, k, v, out, qs, ks, vs, os, idx, order, B, H, Sk, D,
                                             dtype, nq, nk, top_k, sm_scale, gq, gk);
  return launch_status(lcv::launch_attn(p, dtype, (int)D, (hipStream_t)stream),
                       "lcv_bsa_attn_fwd");
}

}  // extern "C"

namespace {
size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }
size_t pooled_bytes(int64_t B, int64_t H, int64_t nb, int64_t D) {
  return align256((size_t)B * H * nb * D * sizeof(float));
}
size_t score_bytes(int64_t B, int64_t H, int64_t nb) {
  return align256((size_t)B * H * nb * nb * sizeof(float));
}
}  // namespace

extern "C" {

size_t lcv_bsa_forward_workspace_bytes(int64_t B, int64_t H, int64_t nb, int64_t D) {
  if (B <= 0 || H <= 0 || nb <= 0 || D <= 0) return 0;
  return 2 * pooled_bytes(B, H, nb, D) + score_bytes(B, H, nb) +
         align256((size_t)B * H * nb * sizeof(int32_t));
}

}  // extern "C"

namespace {

// Validation shared by both forward entry points; fills nb and bs.
int check_forward_args(const void* q, const void* k, const void* v, int dtype, int64_t B,
                       int64_t H, int64_t S, int64_t D, const lcv_bsa_strides& qs,
                       const lcv_bsa_strides& ks, const lcv_bsa_strides& vs, int64_t top_k,
                       float sm_scale, const lcv_bsa_geom& g, const int32_t* idx, const void* out,
                       const lcv_bsa_strides& os, int64_t* nb, int64_t* bs) {
  int64_t nk = 0;
  int st = check_attn_args(q, k, v, out, dtype, B, H, S, S, D, qs, ks, vs, os, top_k, sm_scale, g,
                           g, nb, &nk, bs);
  if (st) return st;
  if (!idx) return fail(LCV_BSA_ERR_INVALID_ARG, "null idx pointer");
  if (top_k > *nb)
    return fail(LCV_BSA_ERR_INVALID_ARG, "top_k=%lld exceeds num_blocks=%lld", (long long)top_k,
                (long long)*nb);
  return check_route(B, H, *nb, *nb, D, true);
}

// pool -> routing -> schedule -> attention on validated arguments.  With a
// score buffer the routing runs as the score GEMM (each staged key chunk
// shared by 64 rows) plus the per-row top-k, score_bh (b, h) slices at a
// time (all of them when the buffer holds B*H slices); without one, as the
// fused select kernel that keeps the scores on chip.  All give the same
// routing.
int run_forward(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H,
                int64_t S, int64_t D, const lcv_bsa_strides& qs, const lcv_bsa_strides& ks,
                const lcv_bsa_strides& vs, int64_t top_k, float sm_scale, const lcv_bsa_geom& g,
                int64_t nb, int64_t bs, float* qbar, float* kbar, float* score, int64_t score_bh,
                int32_t* order, int32_t* idx, void* out, const lcv_bsa_strides& os, hipStream_t s,
                const char* name) {
  char what[96];
  const lcv::Tensor4 ts[2] = {{q, qs.b, qs.h, qs.s}, {k, ks.b, ks.h, ks.s}};
  float* outs[2] = {qbar, kbar};
  const lcv::Geom gg = lcv::make_geom(g);
  snprintf(what, sizeof(what), "%s(pool)", name);
  int st = launch_status(lcv::launch_pool(ts, 2, dtype, (int)B, (int)H, (int)D, (int)nb, (int)bs,
                                          gg, outs, s),
                         what);
  if (st) return st;
  if (score) {
    // Slices [c0, c0 + n) of the B*H (b, h) pairs; the scores of one slice
    // are read by its top-k before the next slice's GEMM rewrites them (one
    // stream).
    for (int64_t c0 = 0; c0 < B * H && !st; c0 += score_bh) {
      const int64_t n = B * H - c0 < score_bh ? B * H - c0 : score_bh;
      snprintf(what, sizeof(what), "%s(scores)", name);
      st = launch_status(lcv::launch_scores(qbar + c0 * nb * D, kbar + c0 * nb * D, 1, (int)n,
                                            (int)nb, (int)nb, (int)D, score, s),
                         what);
      if (st) return st;
      snprintf(what, sizeof(what), "%s(top-k)", name);
      st = launch_status(lcv::launch_topk(score, 1, (int)n, (int)nb, (int)nb, (int)top_k,
                                          idx + c0 * nb * top_k, s),
                         what);
    }
  } else {
    snprintf(what, sizeof(what), "%s(select)", name);
    st = launch_status(lcv::launch_select(qbar, kbar, (int)B, (int)H, (int)nb, (int)nb, (int)D,
                                          (int)top_k, idx, s),
                       what);
  }
  if (st) return st;
  const bool sched = lcv::schedule_supported((int)nb, (int)nb);
  if (sched) {
    snprintf(what, sizeof(what), "%s(schedule)", name);
    st = launch_status(lcv::launch_schedule(idx, (int)(B * H), (int)nb, (int)nb, (int)top_k, order,
                                            s),
                       what);
    if (st) return st;
  }
  const lcv::AttnParams p = make_attn_params(q, k, v, out, qs, ks, vs, os, idx,
                                             sched ? order : nullptr, B, H, S, D, dtype, nb, nb,
                                             top_k, sm_scale, g, g);
  snprintf(what, sizeof(what), "%s(attn)", name);
  return launch_status(lcv::launch_attn(p, dtype, (int)D, s), what);
}

// ---------------------------------------------------------------------------
// Device scratch of lcv_bsa_forward_noalloc: the launch order (one int32 per
// (b, h, q-block)), in a file-scope array that every GPU the library runs on
// holds (its own copy) until the process ends.  The pooled means and block
// scores are staged in the caller's out buffer instead (the attention, the
// last kernel, overwrites every byte of it).  Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device
// address): the device address comes from hipGetSymbolAddress, once per
// device, with that device current, and is kept per device.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = size_t{1} << 20;  // LCV_BSA_NOALLOC_SCRATCH_BYTES
static_assert(kNoAllocScratchBytes == LCV_BSA_NOALLOC_SCRATCH_BYTES, "header and library agree");
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// At most this many score slices (two launches each) in the no-allocation
// routing; beyond it the single fused select launch is the faster route.
constexpr int64_t kMaxScoreSlices = 8;

// Per device: the array's address and an event recorded after each
// uncaptured call's last launch, so that the next call, if it comes on
// another stream, waits for the launch order that call still reads.
struct NoAllocDevice {
  void* scratch = nullptr;
  hipEvent_t done = nullptr;
  hipStream_t done_stream = nullptr;
  bool recorded = false;
};
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;  // held for a whole call: calls from several host threads queue
NoAllocDevice g_noalloc[kMaxDevices];

// Set-up on the first call on each device: resolve the array's address and
// create the ordering event.  That call must not be under stream capture:
// resolving the symbol may load the library's code object onto the device,
// which a capture cannot record.  It is refused there (before any device
// work).  Caller holds g_noalloc_mu.
int noalloc_device(bool capturing, NoAllocDevice** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(LCV_BSA_ERR_LAUNCH, "lcv_bsa_forward_noalloc: hipGetDevice: %s",
                hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(LCV_BSA_ERR_UNSUPPORTED, "lcv_bsa_forward_noalloc: device %d beyond %d", dev,
                kMaxDevices);
  NoAllocDevice& d = g_noalloc[dev];
  if (!d.scratch) {
    if (capturing)
      return fail(LCV_BSA_ERR_UNSUPPORTED,
                  "lcv_bsa_forward_noalloc: the first call on device %d is under stream capture; "
                  "call it once outside capture on that device first", dev);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(LCV_BSA_ERR_LAUNCH, "lcv_bsa_forward_noalloc: hipGetSymbolAddress(scratch) on "
                  "device %d: %s", dev, hipGetErrorString(e));
    if (!d.done && (e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming)) != hipSuccess) {
      d.done = nullptr;
      return fail(LCV_BSA_ERR_LAUNCH, "lcv_bsa_forward_noalloc: hipEventCreate on device %d: %s",
                  dev, hipGetErrorString(e));
    }
    d.scratch = p;
  }
  *out = &d;
  return LCV_BSA_OK;
}

// Bytes from a [B, H, S, D] view's first element to one past its last
// (non-negative strides; 128-bit arithmetic, so no stride overflows it).
unsigned __int128 view_span_bytes(int64_t B, int64_t H, int64_t S, int64_t D,
                                  const lcv_bsa_strides& s, size_t esz) {
  typedef unsigned __int128 u128;
  return ((u128)(B - 1) * (u128)s.b + (u128)(H - 1) * (u128)s.h + (u128)(S - 1) * (u128)s.s +
          (u128)D) * (u128)esz;
}

bool ranges_overlap(const void* a, unsigned __int128 an, const void* b, unsigned __int128 bn) {
  typedef unsigned __int128 u128;
  const u128 x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + bn && y < x + an;
}

// True when the B*H*S*D elements of a [B, H, S, D] view (unit stride along
// D) fill one contiguous range: the strides of the dimensions longer than 1,
// taken in increasing order, are D, D times the first extent, and so on.
bool dense_view(int64_t B, int64_t H, int64_t S, int64_t D, const lcv_bsa_strides& s) {
  int64_t n[3] = {B, H, S}, st[3] = {s.b, s.h, s.s};
  for (int i = 0; i < 3; ++i)
    for (int j = i + 1; j < 3; ++j)
      if (st[j] < st[i]) {
        std::swap(st[i], st[j]);
        std::swap(n[i], n[j]);
      }
  int64_t expect = D;
  for (int i = 0; i < 3; ++i) {
    if (n[i] == 1) continue;
    if (st[i] != expect) return false;
    expect *= n[i];
  }
  return true;
}

}  // namespace

extern "C" {

int lcv_bsa_forward(const void* q, const void* k, const void* v, int dtype, int64_t B, int64_t H,
                    int64_t S, int64_t D, lcv_bsa_strides qs, lcv_bsa_strides ks,
                    lcv_bsa_strides vs, int64_t top_k, float sm_scale, lcv_bsa_geom g,
                    void* workspace, size_t workspace_bytes, int32_t* idx, void* out,
                    lcv_bsa_strides os, void* stream) {
  int64_t nb = 0, bs = 0;
  int st = check_forward_args(q, k, v, dtype, B, H, S, D, qs, ks, vs, top_k, sm_scale, g, idx, out,
                              os, &nb, &bs);
  if (st) return st;
  if (!workspace) return fail(LCV_BSA_ERR_INVALID_ARG, "null workspace pointer");
  const size_t need = lcv_bsa_forward_workspace_bytes(B, H, nb, D);
  if (workspace_bytes < need || ((uintptr_t)workspace & 255u))
    return fail(LCV_BSA_ERR_INVALID_ARG,
                "workspace must be 256-byte aligned and hold %zu bytes (got %zu)", need,
                workspace_bytes);
  const size_t pb = pooled_bytes(B, H, nb, D);
  char* ws = reinterpret_cast<char*>(workspace);
  return run_forward(q, k, v, dtype, B, H, S, D, qs, ks, vs, top_k, sm_scale, g, nb, bs,
                     reinterpret_cast<float*>(ws), reinterpret_cast<float*>(ws + pb),
                     reinterpret_cast<float*>(ws + 2 * pb), B * H,
                     reinterpret_cast<int32_t*>(ws + 2 * pb + score_bytes(B, H, nb)), idx, out, os,
                     (hipStream_t)stream, "lcv_bsa_forward");
}

int lcv_bsa_forward_noalloc(const void* q, const void* k, const void* v, int dtype, int64_t B,
                            int64_t H, int64_t S, int64_t D, lcv_bsa_strides qs,
                            lcv_bsa_strides ks, lcv_bsa_strides vs, int64_t top_k,
                            float sm_scale, lcv_bsa_geom g, int32_t* idx, void* out,
                            lcv_bsa_strides os, void* stream) {
  int64_t nb = 0, bs = 0;
  int st = check_forward_args(q, k, v, dtype, B, H, S, D, qs, ks, vs, top_k, sm_scale, g, idx, out,
                              os, &nb, &bs);
  if (st) return st;
  // Every size, layout and overlap is checked before the device is touched.
  const size_t order_bytes = align256((size_t)B * H * nb * sizeof(int32_t));
  if (order_bytes > kNoAllocScratchBytes)
    return fail(LCV_BSA_ERR_UNSUPPORTED,
                "lcv_bsa_forward_noalloc: the launch order of B=%lld H=%lld num_blocks=%lld needs "
                "%zu bytes, beyond its fixed device scratch of %zu bytes; call lcv_bsa_forward "
                "with a workspace instead",
                (long long)B, (long long)H, (long long)nb, order_bytes, kNoAllocScratchBytes);
  // The pooled means and block scores are staged in out, which the
  // attention overwrites last: out must be one dense range that no input
  // and not idx overlaps.
  if (!dense_view(B, H, S, D, os))
    return fail(LCV_BSA_ERR_LAYOUT,
                "lcv_bsa_forward_noalloc stages the pooled means and block scores in out: out "
                "must be dense (strides b=%lld h=%lld s=%lld leave gaps); call lcv_bsa_forward "
                "with a workspace instead", (long long)os.b, (long long)os.h, (long long)os.s);
  const size_t esz = (size_t)elem_bytes(dtype);
  const size_t out_bytes = (size_t)(B * H * S * D) * esz;
  if (ranges_overlap(out, out_bytes, q, view_span_bytes(B, H, S, D, qs, esz)) ||
      ranges_overlap(out, out_bytes, k, view_span_bytes(B, H, S, D, ks, esz)) ||
      ranges_overlap(out, out_bytes, v, view_span_bytes(B, H, S, D, vs, esz)) ||
      ranges_overlap(out, out_bytes, idx, (size_t)(B * H * nb * top_k) * sizeof(int32_t)))
    return fail(LCV_BSA_ERR_INVALID_ARG,
                "lcv_bsa_forward_noalloc stages the pooled means and block scores in out: out "
                "must not overlap q, k, v or idx");
  const uintptr_t out_addr = (uintptr_t)out, stage_addr = (out_addr + 255) & ~(uintptr_t)255;
  const size_t stage_bytes = out_bytes - (size_t)(stage_addr - out_addr);
  const size_t pb = pooled_bytes(B, H, nb, D);
  if (2 * pb > stage_bytes)  // out holds 64*D elements per block, the means 2*D floats
    return fail(LCV_BSA_ERR_UNSUPPORTED, "lcv_bsa_forward_noalloc: out too small for the means");
  // What is left after the means holds the block scores of score_bh (b, h)
  // slices; the two-kernel routing runs slice by slice when a few slices
  // cover every head (at 720p, H=32, all heads in one slice), else the fused
  // select kernel routes without scores.
  const size_t slice = align256((size_t)nb * nb * sizeof(float));
  const int64_t score_bh = (int64_t)((stage_bytes - 2 * pb) / slice);
  const bool sliced = score_bh > 0 && (B * H + score_bh - 1) / score_bh <= kMaxScoreSlices;
  const hipStream_t s = (hipStream_t)stream;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cs);
  if (e != hipSuccess)
    return fail(LCV_BSA_ERR_LAUNCH, "lcv_bsa_forward_noalloc: hipStreamIsCapturing: %s",
                hipGetErrorString(e));
  const bool capturing = cs != hipStreamCaptureStatusNone;
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  NoAllocDevice* d = nullptr;
  if ((st = noalloc_device(capturing, &d))) return st;
  // An uncaptured call on another stream than the previous uncaptured call
  // waits for that call's work: both use this device's launch order.
  if (!capturing && d->recorded && d->done_stream != s &&
      (e = hipStreamWaitEvent(s, d->done, 0)) != hipSuccess)
    return fail(LCV_BSA_ERR_LAUNCH, "lcv_bsa_forward_noalloc: hipStreamWaitEvent: %s",
                hipGetErrorString(e));
  char* stage = reinterpret_cast<char*>(stage_addr);
  st = run_forward(q, k, v, dtype, B, H, S, D, qs, ks, vs, top_k, sm_scale, g, nb, bs,
                   reinterpret_cast<float*>(stage), reinterpret_cast<float*>(stage + pb),
                   sliced ? reinterpret_cast<float*>(stage + 2 * pb) : nullptr, score_bh,
                   reinterpret_cast<int32_t*>(d->scratch), idx, out, os, s,
                   "lcv_bsa_forward_noalloc");
  if (!capturing) {
    if ((e = hipEventRecord(d->done, s)) != hipSuccess) {
      d->recorded = false;
      if (!st)
        st = fail(LCV_BSA_ERR_LAUNCH, "lcv_bsa_forward_noalloc: hipEventRecord: %s",
                  hipGetErrorString(e));
    } else {
      d->recorded = true;
      d->done_stream = s;
    }
  }
  return st;
}

int lcv_bsa_block_rows(const void* x, const void* a, int dtype, int64_t B, int64_t N, int64_t C,
                       int64_t frames, const float* gate, const float* shift, const float* scale,
                       const void* ln_weight, const void* ln_bias, float eps, void* x_out,
                       void* n_out, void* stream) {
  if (!x) return fail(LCV_BSA_ERR_INVALID_ARG, "null x");
  if (dtype != LCV_BSA_F16 && dtype != LCV_BSA_BF16)
    return fail(LCV_BSA_ERR_DTYPE, "block row ops take fp16 or bf16 (got dtype %d)", dtype);
  if (B <= 0 || N <= 0 || C <= 0 || frames <= 0 || N % frames)
    return fail(LCV_BSA_ERR_SHAPE, "B, N, C, frames must be positive with N %% frames == 0 "
                "(B=%lld N=%lld C=%lld frames=%lld)", (long long)B, (long long)N, (long long)C,
                (long long)frames);
  if (!lcv::rows_supported(dtype, (int)C))
    return fail(LCV_BSA_ERR_UNSUPPORTED, "block row ops need C %% 8 == 0 and C <= 8192 (C=%lld)",
                (long long)C);
  if (B * N > kI32Max / 2 || B * N * C > (int64_t{1} << 40))
    return fail(LCV_BSA_ERR_UNSUPPORTED, "tensor too large");
  if (gate && !a) return fail(LCV_BSA_ERR_INVALID_ARG, "gate needs a residual input a");
  if (x_out && !a) return fail(LCV_BSA_ERR_INVALID_ARG, "x_out needs a residual input a");
  if ((!shift) != (!scale)) return fail(LCV_BSA_ERR_INVALID_ARG, "shift and scale go together");
  if ((!ln_weight) != (!ln_bias))
    return fail(LCV_BSA_ERR_INVALID_ARG, "ln_weight and ln_bias go together");
  if ((shift || ln_weight) && !n_out)
    return fail(LCV_BSA_ERR_INVALID_ARG, "normalisation parameters given without n_out");
  if (!x_out && !n_out) return fail(LCV_BSA_ERR_INVALID_ARG, "nothing to write");
  const void* ptrs[] = {x, a, gate, shift, scale, ln_weight, ln_bias, x_out, n_out};
  for (const void* q : ptrs)
    if ((uintptr_t)q % 16) return fail(LCV_BSA_ERR_LAYOUT, "all tensors must be 16-byte aligned");
  return launch_status(lcv::launch_rows(x, a, gate, shift, scale, ln_weight, ln_bias, x_out, n_out,
                                        dtype, (int)(B * N), (int)C, (int)N, (int)(N / frames),
                                        (int)frames, eps, (hipStream_t)stream),
                       "lcv_bsa_block_rows");
}

int lcv_bsa_block_swiglu(const void* h13, int dtype, int64_t rows, int64_t hidden, void* out,
                         void* stream) {
  if (!h13 || !out) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  if (dtype != LCV_BSA_F16 && dtype != LCV_BSA_BF16)
    return fail(LCV_BSA_ERR_DTYPE, "swiglu takes fp16 or bf16 (got dtype %d)", dtype);
  if (rows <= 0 || hidden <= 0 || hidden % 8 || rows * hidden > (int64_t{1} << 40) ||
      hidden > kI32Max)
    return fail(LCV_BSA_ERR_SHAPE, "swiglu needs rows > 0 and hidden a positive multiple of 8");
  if ((uintptr_t)h13 % 16 || (uintptr_t)out % 16)
    return fail(LCV_BSA_ERR_LAYOUT, "swiglu tensors must be 16-byte aligned");
  return launch_status(lcv::launch_swiglu(h13, out, dtype, rows, (int)hidden, (hipStream_t)stream),
                       "lcv_bsa_block_swiglu");
}

int lcv_bsa_head_rms_norm(const void* x, int dtype, int64_t B, int64_t H, int64_t S, int64_t D,
                          lcv_bsa_strides xs, const void* weight, float eps, void* out,
                          lcv_bsa_strides os, void* stream) {
  if (!x || !out) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  if (dtype != LCV_BSA_F16 && dtype != LCV_BSA_BF16)
    return fail(LCV_BSA_ERR_DTYPE, "head RMSNorm takes fp16 or bf16 (got dtype %d)", dtype);
  if (!(D == 64 || D == 128)) return fail(LCV_BSA_ERR_UNSUPPORTED, "head RMSNorm needs D in {64, 128}");
  if (B <= 0 || H <= 0 || S <= 0 || B * H * S > kI32Max / 2)
    return fail(LCV_BSA_ERR_SHAPE, "B, H, S must be positive and B*H*S < 2^30");
  if (!std::isfinite(eps) || eps < 0.0f) return fail(LCV_BSA_ERR_INVALID_ARG, "eps must be >= 0");
  int st = 0;
  if ((st = check_strides("x", xs, D)) || (st = check_strides("out", os, D))) return st;
  if (!vec_aligned(x, xs, 8) || !vec_aligned(out, os, 8) || (uintptr_t)weight % 16)
    return fail(LCV_BSA_ERR_LAYOUT, "rows and weight must start on 16-byte boundaries");
  const int64_t xst[3] = {xs.b, xs.s, xs.h}, ost[3] = {os.b, os.s, os.h};
  return launch_status(lcv::launch_head_norm(x, xst, out, ost, weight, dtype, (int)B, (int)S,
                                             (int)H, (int)D, eps, (hipStream_t)stream),
                       "lcv_bsa_head_rms_norm");
}

int lcv_bsa_token_blocks(lcv_bsa_geom g, int32_t* out, void* stream) {
  if (!out) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  int64_t nb = 0, bs = 0;
  const int64_t S = g.T * g.Hl * g.Wl;
  int st = check_geom(1, 1, S > 0 ? S : 1, 1, g, &nb, &bs);
  if (st) return st;
  return launch_status(lcv::launch_token_blocks(lcv::make_geom(g), (int)g.T, out,
                                                (hipStream_t)stream),
                       "lcv_bsa_token_blocks");
}

int lcv_bsa_token_pair_mask(const int32_t* idx, int64_t B, int64_t H, int64_t nq,
                            int64_t top_k, const int32_t* token_block, int64_t S,
                            int64_t num_kv_blocks, uint8_t* mask, void* stream) {
  if (!idx || !token_block || !mask) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  if (B <= 0 || H <= 0 || nq <= 0 || top_k <= 0 || S <= 0 || num_kv_blocks <= 0)
    return fail(LCV_BSA_ERR_INVALID_ARG, "B, H, nq, top_k, S, num_kv_blocks must be positive");
  if (S > kI32Max || nq > kI32Max || num_kv_blocks > kI32Max || B * H * nq * top_k > kI32Max * 8 ||
      B * H * S * S > ((int64_t)1 << 34))
    return fail(LCV_BSA_ERR_UNSUPPORTED, "token-pair mask of %lld entries is too large",
                (long long)(B * H * S * S));
  return launch_status(lcv::launch_pair_mask(idx, (int)B, (int)H, (int)nq, (int)top_k,
                                             token_block, (int)S, (int)num_kv_blocks, mask,
                                             (hipStream_t)stream),
                       "lcv_bsa_token_pair_mask");
}

int lcv_bsa_permute_block_major(const void* x, int dtype, int64_t B, int64_t H, int64_t S,
                                int64_t D, lcv_bsa_geom g, int inverse, void* out,
                                void* stream) {
  if (!x || !out) return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  if (!dtype_ok(dtype)) return fail(LCV_BSA_ERR_DTYPE, "unknown dtype %d", dtype);
  int64_t nb = 0, bs = 0;
  int st = check_geom(B, H, S, D, g, &nb, &bs);
  if (st) return st;
  if (B * H * S * D > ((int64_t)1 << 38))
    return fail(LCV_BSA_ERR_UNSUPPORTED, "tensor too large");
  return launch_status(lcv::launch_permute(x, elem_bytes(dtype), (int)B, (int)H, (int)S, (int)D,
                                           lcv::make_geom(g), inverse ? 1 : 0, out,
                                           (hipStream_t)stream),
                       "lcv_bsa_permute_block_major");
}


int64_t lcv_bsa_rope_table_len(int64_t D, lcv_bsa_grid rope) {
  if (!(D == 64 || D == 128) || rope.T <= 0 || rope.Hl <= 0 || rope.Wl <= 0) return 0;
  const int64_t dt = D - 4 * (D / 6), dh = 2 * (D / 6), dw = 2 * (D / 6);
  const int64_t len = rope.T * dt + rope.Hl * dh + rope.Wl * dw;  // cos + sin, half dims each
  return len <= lcv::kMaxRopeTable ? len : 0;
}

int lcv_bsa_prepare_qk(const void* q_in, const void* k_in, int dtype, int64_t B, int64_t H,
                       int64_t S, int64_t D, lcv_bsa_strides qis, lcv_bsa_strides kis,
                       const void* q_weight, const void* k_weight, float eps, lcv_bsa_grid rope,
                       const float* rope_table, int64_t rope_table_len, lcv_bsa_geom g,
                       void* q_out, void* k_out, lcv_bsa_strides qos, lcv_bsa_strides kos,
                       float* qbar, float* kbar, void* stream) {
  if (!q_in || !k_in || !q_out || !k_out || !qbar || !kbar || !rope_table)
    return fail(LCV_BSA_ERR_INVALID_ARG, "null pointer");
  if (!dtype_ok(dtype)) return fail(LCV_BSA_ERR_DTYPE, "unknown dtype %d", dtype);
  if (!lcv::prep_supported(dtype, (int)D))
    return fail(LCV_BSA_ERR_UNSUPPORTED, "prepare_qk supports fp16/bf16 with D in {64, 128}");
  int64_t nb = 0, bs = 0;
  int st = check_geom(B, H, S, D, g, &nb, &bs);
  if (st) return st;
  if (bs != 64)
    return fail(LCV_BSA_ERR_UNSUPPORTED, "prepare_qk requires 64-token blocks (got %lld)",
                (long long)bs);
  if (rope.T <= 0 || rope.Hl <= 0 || rope.Wl <= 0 || rope.T * rope.Hl * rope.Wl != S)
    return fail(LCV_BSA_ERR_SHAPE, "RoPE grid (%lld, %lld, %lld) must be positive with product S=%lld",
                (long long)rope.T, (long long)rope.Hl, (long long)rope.Wl, (long long)S);
  if (S > lcv::kPrepMaxTokens)
    return fail(LCV_BSA_ERR_UNSUPPORTED, "prepare_qk supports at most %lld tokens (S=%lld)",
                (long long)lcv::kPrepMaxTokens, (long long)S);
  const int64_t need = lcv_bsa_rope_table_len(D, rope);
  if (need == 0)
    return fail(LCV_BSA_ERR_UNSUPPORTED, "RoPE table for this grid exceeds %d floats",
                lcv::kMaxRopeTable);
  if (rope_table_len != need)
    return fail(LCV_BSA_ERR_INVALID_ARG, "rope_table_len=%lld, expected %lld",
                (long long)rope_table_len, (long long)need);
  if (!std::isfinite(eps) || eps < 0.0f) return fail(LCV_BSA_ERR_INVALID_ARG, "eps must be >= 0");
  if ((st = check_strides("q_in", qis, D)) || (st = check_strides("k_in", kis, D)) ||
      (st = check_strides("q_out", qos, D)) || (st = check_strides("k_out", kos, D)))
    return st;
  if (!vec_aligned(q_in, qis, 8) || !vec_aligned(k_in, kis, 8) || !vec_aligned(q_out, qos, 8) ||
      !vec_aligned(k_out, kos, 8))
    return fail(LCV_BSA_ERR_LAYOUT, "q/k rows must start on 16-byte boundaries");
  if ((uintptr_t)q_weight % 16 || (uintptr_t)k_weight % 16 || (uintptr_t)qbar % 16 ||
      (uintptr_t)kbar % 16)
    return fail(LCV_BSA_ERR_LAYOUT, "norm weights and block means must be 16-byte aligned");
  const lcv::Tensor4 in[2] = {{q_in, qis.b, qis.h, qis.s}, {k_in, kis.b, kis.h, kis.s}};
  const lcv::Tensor4 out[2] = {{q_out, qos.b, qos.h, qos.s}, {k_out, kos.b, kos.h, kos.s}};
  const void* w[2] = {q_weight, k_weight};
  float* means[2] = {qbar, kbar};
  const int32_t grid[3] = {(int32_t)rope.T, (int32_t)rope.Hl, (int32_t)rope.Wl};
  const int32_t dims[2] = {(int32_t)(D - 4 * (D / 6)), (int32_t)(2 * (D / 6))};
  return launch_status(lcv::launch_prep(in, out, w, means, dtype, (int)B, (int)H, (int)D, (int)nb,
                                        lcv::make_geom(g), grid, dims, rope_table, (int)need, eps,
                                        (hipStream_t)stream),
                       "lcv_bsa_prepare_qk");
}

}  // extern "C"
