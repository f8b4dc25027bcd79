// extern "C" entry points of liblizard_hip.so; declarations and the
// reference code each one replaces are in include/lizard_hip.h.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <string>

#include "../../include/lizard_hip.h"
#include "common.hpp"

namespace lz {
hipError_t launch_gla_fwd(const void* fq, const void* fk, const void* v, const float* lg, void* y,
                          int B, int H, int L, int F, int D, int gate_per_head, int KG, float* ws,
                          float* final_state, float* raw_den, hipStream_t st);
hipError_t launch_gla_fwd_phi(const void* q, const void* wq, const void* fk, const void* v,
                              const float* lg, void* y, int B, int H, int L, int gate, int KG,
                              float* ws, float* final_state, hipStream_t st);
hipError_t launch_gla_decode(const void* fq, const void* fk, const void* v, const float* lg,
                             float* state, void* y, int B, int H, int F, int D,
                             int gate_per_head, int KG, hipStream_t st);
size_t gla_fwd_workspace(int B, int H, int L, int F, int D);
hipError_t gla_fwd_prepare();
bool gla_dims_supported(int F, int D);
struct GlaTiles {
  int nF, Ft, nD, Dt;
  bool native() const { return nF == 1 && nD == 1; }
};
GlaTiles gla_tiles(int F, int D);
size_t gla_fwd_workspace_any(int B, int H, int L, int F, int D);
size_t gla_bwd_workspace_any(int B, int H, int L, int F, int D, int gate_per_head);
hipError_t launch_gla_fwd_any(const void* fq, const void* fk, const void* v, const float* lg,
                              void* y, int B, int H, int L, int F, int D, int gate_per_head,
                              int KG, void* ws, hipStream_t st);
hipError_t launch_gla_bwd_any(const void* fq, const void* fk, const void* v, const float* lg,
                              const void* dy, void* dfq, void* dfk, void* dv, float* dlg,
                              bool grad_bf16, int B, int H, int L, int F, int D,
                              int gate_per_head, int KG, const float* fwd_ws, void* ws,
                              hipStream_t st);
int swa_padded_dim(int d);
int swa_row_blocks(int L);
hipError_t launch_swa_fwd(const void* q, const void* k, const void* v, const float* meta,
                          int n_meta, void* y, float* lse, int BH, int L, int d, int W,
                          float scale, int KG, hipStream_t st);
constexpr int SWA_DEC_MAX_W = 8192;
hipError_t launch_swa_decode(const void* q, const void* k_cache, const void* v_cache,
                             const float* meta, int n_meta, void* y, int BH, int W, int d,
                             int pos, float scale, int KG, hipStream_t st);
hipError_t launch_swa_bwd(const void* q, const void* k, const void* v, const float* meta,
                          int n_meta, const float* lse, const void* dy, void* dq, void* dk,
                          void* dv, bool grad_bf16, float* delta, float* dmeta_part,
                          float* dmeta, int BH, int L, int d, int W, float scale, int KG,
                          hipStream_t st);
constexpr int MAX_META = LZ_SWA_MAX_META;
bool prologue_dims_supported(int hd, int f, bool bf16_in);
size_t prologue_bwd_workspace(int B, int L, int H, int Hkv, int hd, int f);
hipError_t launch_prologue_fwd(const void* q, const void* k, const void* v, const void* wq,
                               const void* wk, const void* cos, const void* sin, void* fq,
                               void* fk, void* qr, void* kr, void* vo, bool bf16_in, int B, int L,
                               int H, int Hkv, int hd, int f, int cos_bstride, hipStream_t st);
hipError_t launch_prologue_bwd(const void* q, const void* k, const void* wq, const void* wk,
                               const void* cos, const void* sin, const void* dfq,
                               const void* dfk, const void* dqr, const void* dkr,
                               const void* dv, const void* dv2, void* dq, void* dk, void* dvo,
                               float* dwq, float* dwk, bool bf16_in, int B, int L, int H, int Hkv,
                               int hd, int f, int cos_bstride, float* ws, hipStream_t st);
size_t combine_bwd_workspace();
hipError_t launch_combine_fwd(const void* yg, const void* ys, const float* alpha, void* out,
                              bool bf16_out, int B, int H, int L, int hd, hipStream_t st);
hipError_t launch_combine_bwd(const void* dout, const void* ys, const float* alpha, void* dyg,
                              void* dys, float* dalpha, bool bf16_out, int B, int H, int L,
                              int hd, float* ws, hipStream_t st);

}  // namespace lz

static thread_local std::string g_err;

static int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
static int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

static int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_err.clear();
    return 0;
  }
  return fail((int)e, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

static bool pow2_at_least_16(int c) { return c >= 16 && (c & (c - 1)) == 0; }

extern "C" int lz_abi_version(void) { return LZ_ABI_VERSION; }

extern "C" const char* lz_last_error(void) { return g_err.c_str(); }

// The kernels address each (batch, head) slab through a buffer resource with a
// 32-bit range and 32-bit offsets, and index rows (batch, head, token) with
// 32-bit ints: a slab of fp32 rows must stay under 2 GiB, and B*H*L under 2^31.
static int check_extent(const char* what, int batch, int heads, int length, int width) {
  if ((long long)length * width * 4 >= (1LL << 31))
    return fail(1, "%s: length %d x width %d exceeds the 2 GiB (batch, head) slab limit", what,
                length, width);
  if ((long long)batch * heads * length > (1LL << 31) - (1LL << 20))
    return fail(1, "%s: B*H*L = %lld rows exceeds the 2^31 - 2^20 row limit", what,
                (long long)batch * heads * length);
  return 0;
}

// `native`: the entry point runs the walks directly (prefill, decode, the
// no-allocation forward), so F and D must be within their own sizes; the
// forward and backward take any F and D (tiles of the walks past them).
static int check_gla(const void* fq, const void* fk, const void* v, const float* lg, int batch,
                     int heads, int length, int nf, int nd, int chunk, bool native) {
  if (!fq || !fk || !v || !lg) return fail(1, "gla: null input pointer");
  if (batch <= 0 || heads <= 0 || length <= 0 || nf <= 0 || nd <= 0)
    return fail(1, "gla: sizes must be positive (B=%d H=%d L=%d F=%d D=%d)", batch, heads,
                length, nf, nd);
  if (!pow2_at_least_16(chunk)) return fail(1, "gla: chunk must be a power of two >= 16, got %d", chunk);
  if (native && !lz::gla_dims_supported(nf, nd))
    return fail(1, "gla: unsupported feature/value dims F=%d D=%d for this entry point (need "
                   "F<=256, D<=128, and D<=64 when F>128)", nf, nd);
  if (nf > LZ_GLA_MAX_DIM || nd > LZ_GLA_MAX_DIM)
    return fail(1, "gla: feature/value dims F=%d D=%d beyond %d unsupported", nf, nd,
                LZ_GLA_MAX_DIM);
  return check_extent("gla", batch, heads, length, nf > nd ? nf : nd);
}

// kv_heads heads of k-side operands (fk and v; k and v), each shared by
// heads / kv_heads consecutive query heads (grouped-query attention)
static int check_kv_heads(const char* what, int heads, int kv_heads) {
  if (kv_heads <= 0 || heads % kv_heads)
    return fail(1, "%s: kv_heads (%d) must be positive and divide heads (%d)", what, kv_heads,
                heads);
  return 0;
}

static_assert(LZ_GATE_PER_HEAD == lz::GATE_PER_HEAD && LZ_GATE_LOGIT == lz::GATE_LOGIT &&
                  LZ_GLA_NO_REUSE == lz::GATE_NO_REUSE,
              "gate mode bits");

// gate_mode: LZ_GATE_PER_HEAD, LZ_GATE_LOGIT and LZ_GLA_NO_REUSE bits,
// nothing else (the entry points that do not walk forward ignore the hint)
static int check_gate_mode(const char* what, int gate_mode) {
  if (gate_mode & ~(LZ_GATE_PER_HEAD | LZ_GATE_LOGIT | LZ_GLA_NO_REUSE))
    return fail(1, "%s: gate_mode %d has bits other than LZ_GATE_PER_HEAD (1), "
                   "LZ_GATE_LOGIT (2) and LZ_GLA_NO_REUSE (4)", what, gate_mode);
  return 0;
}

extern "C" size_t lz_gla_fwd_workspace_bytes(int batch, int heads, int length, int nf, int nd,
                                             int gate_mode, int chunk) {
  (void)gate_mode; (void)chunk;
  if (batch <= 0 || heads <= 0 || length <= 0 || nf <= 0 || nd <= 0 || nf > LZ_GLA_MAX_DIM ||
      nd > LZ_GLA_MAX_DIM)
    return 0;
  return lz::gla_fwd_workspace_any(batch, heads, length, nf, nd);
}

extern "C" int lz_gla_fwd(const void* fq, const void* fk, const void* v, const float* log_gamma,
                          void* y, int batch, int heads, int kv_heads, int length, int nf, int nd,
                          int gate_mode, int chunk, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (int rc = check_gla(fq, fk, v, log_gamma, batch, heads, length, nf, nd, chunk, false))
    return rc;
  if (int rc = check_kv_heads("gla_fwd", heads, kv_heads)) return rc;
  if (int rc = check_gate_mode("gla_fwd", gate_mode)) return rc;
  if (!y) return fail(1, "gla_fwd: null output pointer");
  const size_t need = lz::gla_fwd_workspace_any(batch, heads, length, nf, nd);
  if (need && (!workspace || workspace_bytes < need))
    return fail(1, "gla_fwd: workspace of %zu bytes given, %zu needed", workspace_bytes, need);
  return hip_status(lz::launch_gla_fwd_any(fq, fk, v, log_gamma, y, batch, heads, length, nf, nd,
                                           gate_mode, heads / kv_heads, workspace,
                                           (hipStream_t)stream),
                    "gla_fwd");
}

extern "C" int lz_gla_prefill(const void* fq, const void* fk, const void* v,
                              const float* log_gamma, void* y, float* state, int batch, int heads,
                              int kv_heads, int length, int nf, int nd, int gate_mode,
                              int chunk, void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_gla(fq, fk, v, log_gamma, batch, heads, length, nf, nd, chunk, true))
    return rc;
  if (int rc = check_kv_heads("gla_prefill", heads, kv_heads)) return rc;
  if (int rc = check_gate_mode("gla_prefill", gate_mode)) return rc;
  if (!y || !state) return fail(1, "gla_prefill: null output pointer");
  const size_t need = lz::gla_fwd_workspace(batch, heads, length, nf, nd);
  if (need && (!workspace || workspace_bytes < need))
    return fail(1, "gla_prefill: workspace of %zu bytes given, %zu needed", workspace_bytes,
                need);
  return hip_status(lz::launch_gla_fwd(fq, fk, v, log_gamma, y, batch, heads, length, nf, nd,
                                       gate_mode, heads / kv_heads, (float*)workspace,
                                       state, nullptr, (hipStream_t)stream),
                    "gla_prefill");
}

extern "C" int lz_gla_fwd_phi(const void* q, const void* wq, const void* fk, const void* v,
                              const float* log_gamma, void* y, float* state, int batch, int heads,
                              int kv_heads, int length, int head_dim, int feature_dim,
                              int gate_mode, int chunk, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (head_dim != 64 || feature_dim != 128)
    return fail(1, "gla_fwd_phi: head_dim %d x feature_dim %d unsupported (the walk forms the "
                   "feature map at head_dim 64, feature_dim 128)", head_dim, feature_dim);
  const int nf = 2 * feature_dim, nd = head_dim;
  if (int rc = check_gla(fk, fk, v, log_gamma, batch, heads, length, nf, nd, chunk, true))
    return rc;
  if (int rc = check_kv_heads("gla_fwd_phi", heads, kv_heads)) return rc;
  if (int rc = check_gate_mode("gla_fwd_phi", gate_mode)) return rc;
  if (!q || !wq || !y) return fail(1, "gla_fwd_phi: null q, wq or output pointer");
  if ((size_t)length * heads * head_dim * 2 >= ((size_t)1 << 31))
    return fail(1, "gla_fwd_phi: a batch row of q (%d x %d x %d bf16) must stay under 2 GiB",
                length, heads, head_dim);
  const size_t need = lz::gla_fwd_workspace(batch, heads, length, nf, nd);
  if (need && (!workspace || workspace_bytes < need))
    return fail(1, "gla_fwd_phi: workspace of %zu bytes given, %zu needed", workspace_bytes,
                need);
  return hip_status(lz::launch_gla_fwd_phi(q, wq, fk, v, log_gamma, y, batch, heads, length,
                                           gate_mode, heads / kv_heads, (float*)workspace,
                                           state, (hipStream_t)stream),
                    "gla_fwd_phi");
}

extern "C" int lz_gla_decode_step(const void* fq, const void* fk, const void* v,
                                  const float* log_gamma, float* state, void* y, int batch,
                                  int heads, int kv_heads, int nf, int nd, int gate_mode,
                                  void* stream) {
  if (int rc = check_gla(fq, fk, v, log_gamma, batch, heads, 1, nf, nd, 64, true)) return rc;
  if (int rc = check_kv_heads("gla_decode_step", heads, kv_heads)) return rc;
  if (int rc = check_gate_mode("gla_decode_step", gate_mode)) return rc;
  if (!state || !y) return fail(1, "gla_decode_step: null state or output pointer");
  return hip_status(lz::launch_gla_decode(fq, fk, v, log_gamma, state, y, batch, heads, nf, nd,
                                          gate_mode, heads / kv_heads,
                                          (hipStream_t)stream),
                    "gla_decode_step");
}

extern "C" size_t lz_gla_bwd_workspace_bytes(int batch, int heads, int length, int nf, int nd,
                                             int gate_mode, int chunk) {
  (void)chunk;
  if (batch <= 0 || heads <= 0 || length <= 0 || nf <= 0 || nd <= 0 || nf > LZ_GLA_MAX_DIM ||
      nd > LZ_GLA_MAX_DIM)
    return 0;
  return lz::gla_bwd_workspace_any(batch, heads, length, nf, nd, gate_mode);
}

extern "C" int lz_gla_bwd(const void* fq, const void* fk, const void* v, const float* log_gamma,
                          const void* dy, void* dfq, void* dfk, void* dv, float* dlog_gamma,
                          int grad_bf16, int batch, int heads, int kv_heads, int length, int nf,
                          int nd, int gate_mode, int chunk, const void* fwd_workspace,
                          size_t fwd_workspace_bytes, void* workspace, size_t workspace_bytes,
                          void* stream) {
  if (int rc = check_gla(fq, fk, v, log_gamma, batch, heads, length, nf, nd, chunk, false))
    return rc;
  if (int rc = check_kv_heads("gla_bwd", heads, kv_heads)) return rc;
  if (int rc = check_gate_mode("gla_bwd", gate_mode)) return rc;
  if (!dy || !dfq || !dfk || !dv || !dlog_gamma) return fail(1, "gla_bwd: null pointer");
  const size_t need =
      lz::gla_bwd_workspace_any(batch, heads, length, nf, nd, gate_mode);
  if (!workspace || workspace_bytes < need)
    return fail(1, "gla_bwd: workspace of %zu bytes given, %zu needed", workspace_bytes, need);
  // the forward's workspace, if the caller kept it, already holds the state
  // entering each segment; otherwise the backward recomputes it (always for
  // sizes past the walks', whose forward workspace holds tiles instead)
  const bool native = lz::gla_dims_supported(nf, nd);
  const size_t fneed = native ? lz::gla_fwd_workspace(batch, heads, length, nf, nd) : 0;
  const float* fws = nullptr;
  if (fwd_workspace && fneed) {
    if (fwd_workspace_bytes < fneed)
      return fail(1, "gla_bwd: forward workspace of %zu bytes given, %zu needed",
                  fwd_workspace_bytes, fneed);
    fws = (const float*)fwd_workspace;
  }
  return hip_status(lz::launch_gla_bwd_any(fq, fk, v, log_gamma, dy, dfq, dfk, dv, dlog_gamma,
                                           grad_bf16 != 0, batch, heads, length, nf, nd,
                                           gate_mode, heads / kv_heads, fws,
                                           workspace, (hipStream_t)stream),
                    "gla_bwd");
}

// ---------------------------------------------------------------------------
// GLA forward without allocation: the segment records in a static array
// ---------------------------------------------------------------------------
// `scratch` holds the state records of lz_gla_fwd_noalloc's segment split
// (the only device memory the forward needs beyond its inputs and output).
// Its size covers every split the forward makes on a whole MI355X: the
// largest, 64.75 MiB, is F = 256, D = 64 at B*H = 255.  Every GPU the library
// runs on holds its own copy until the process ends.
static_assert(LZ_GLA_FWD_NOALLOC_MAX_BYTES % 256 == 0, "scratch size");
static __device__ __align__(256) float scratch[LZ_GLA_FWD_NOALLOC_MAX_BYTES / sizeof(float)];

// Device address of the current device's copy of `scratch`, looked up once
// per device with that device current.  In host code the array's name is
// only a handle the runtime resolves; kernels get this address instead.
static int scratch_address(float** out) {
  constexpr int MAXDEV = 64;
  static std::once_flag once[MAXDEV];
  static float* addr[MAXDEV];
  static hipError_t status[MAXDEV];
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess)
    return hip_status(e, "gla_fwd_noalloc: hipGetDevice");
  if (dev < 0 || dev >= MAXDEV)
    return fail(1, "gla_fwd_noalloc: device index %d beyond the %d this library tracks", dev,
                MAXDEV);
  std::call_once(once[dev], [dev] {
    void* p = nullptr;
    status[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    addr[dev] = static_cast<float*>(p);
  });
  if (status[dev] != hipSuccess)
    return hip_status(status[dev], "gla_fwd_noalloc: hipGetSymbolAddress(scratch)");
  if (!addr[dev]) return fail(1, "gla_fwd_noalloc: no device address for the scratch array");
  *out = addr[dev];
  return 0;
}

// The no-allocation forward's set-up on the current device, once per device:
// the scratch array's address and the LDS limits of the kernels it launches
// (hipFuncSetAttribute, which the other entry points make on their first
// launch of each kernel).  lz_init makes it eagerly.  Each call still makes
// hipGetDevice calls here and in device_geom, and hipGetLastError after its
// launches.
static int noalloc_setup(float** ws) {
  if (int rc = scratch_address(ws)) return rc;
  constexpr int MAXDEV = 64;
  static std::once_flag once[MAXDEV];
  static hipError_t status[MAXDEV];
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess)
    return hip_status(e, "gla_fwd_noalloc: hipGetDevice");
  std::call_once(once[dev], [dev] { status[dev] = lz::gla_fwd_prepare(); });
  return hip_status(status[dev], "gla_fwd_noalloc: LDS limits of the forward kernels");
}

extern "C" int lz_init(void) {
  float* ws = nullptr;
  return noalloc_setup(&ws);
}

extern "C" int lz_gla_fwd_noalloc(const void* fq, const void* fk, const void* v,
                                  const float* log_gamma, void* y, int batch, int heads,
                                  int kv_heads, int length, int nf, int nd, int gate_mode,
                                  int chunk, void* stream) {
  if (int rc = check_gla(fq, fk, v, log_gamma, batch, heads, length, nf, nd, chunk, true))
    return rc;
  if (int rc = check_kv_heads("gla_fwd_noalloc", heads, kv_heads)) return rc;
  if (int rc = check_gate_mode("gla_fwd_noalloc", gate_mode)) return rc;
  if (!y) return fail(1, "gla_fwd_noalloc: null output pointer");
  const size_t need = lz::gla_fwd_workspace(batch, heads, length, nf, nd);
  if (need > (size_t)LZ_GLA_FWD_NOALLOC_MAX_BYTES)
    return fail(1, "gla_fwd_noalloc: these sizes need %zu bytes of segment records, more than "
                   "the %zu-byte static scratch (use lz_gla_fwd with a workspace)",
                need, (size_t)LZ_GLA_FWD_NOALLOC_MAX_BYTES);
  float* ws = nullptr;
  if (int rc = noalloc_setup(&ws)) return rc;
  if (!need) ws = nullptr;
  return hip_status(lz::launch_gla_fwd(fq, fk, v, log_gamma, y, batch, heads, length, nf, nd,
                                       gate_mode, heads / kv_heads, ws, nullptr,
                                       nullptr, (hipStream_t)stream),
                    "gla_fwd_noalloc");
}

static int check_swa(const void* q, const void* k, const void* v, const float* meta, int n_meta,
                     int batch, int heads, int length, int dim, int window) {
  if (!q || !k || !v) return fail(1, "swa: null input pointer");
  if (n_meta < 0 || n_meta > lz::MAX_META)
    return fail(1, "swa: n_meta must be in [0, %d], got %d", lz::MAX_META, n_meta);
  if (n_meta > 0 && !meta) return fail(1, "swa: null meta pointer");
  if (batch <= 0 || heads <= 0 || length <= 0 || dim <= 0)
    return fail(1, "swa: sizes must be positive (B=%d H=%d L=%d d=%d)", batch, heads, length, dim);
  if (window <= 0) return fail(1, "swa: window must be positive, got %d", window);
  if (lz::swa_padded_dim(dim) < 0) return fail(1, "swa: head dim %d > 256 unsupported", dim);
  return check_extent("swa", batch, heads, length, dim);
}

extern "C" int lz_swa_fwd(const void* q, const void* k, const void* v, const float* meta,
                          int n_meta, void* y, float* lse, int batch, int heads, int kv_heads,
                          int length, int dim, int window, float scale, void* stream) {
  if (int rc = check_swa(q, k, v, meta, n_meta, batch, heads, length, dim, window)) return rc;
  if (int rc = check_kv_heads("swa_fwd", heads, kv_heads)) return rc;
  if (!y || !lse) return fail(1, "swa_fwd: null output pointer");
  return hip_status(lz::launch_swa_fwd(q, k, v, meta, n_meta, y, lse, batch * heads, length, dim,
                                       window, scale, heads / kv_heads, (hipStream_t)stream),
                    "swa_fwd");
}

extern "C" int lz_swa_decode_step(const void* q, const void* k_cache, const void* v_cache,
                                  const float* meta, int n_meta, void* y, int batch, int heads,
                                  int kv_heads, int window, int dim, int pos, float scale,
                                  void* stream) {
  if (int rc = check_swa(q, k_cache, v_cache, meta, n_meta, batch, heads, 1, dim, window))
    return rc;
  if (int rc = check_kv_heads("swa_decode_step", heads, kv_heads)) return rc;
  if (!y) return fail(1, "swa_decode_step: null output pointer");
  if (window > lz::SWA_DEC_MAX_W)
    return fail(1, "swa_decode_step: window %d > %d unsupported", window, lz::SWA_DEC_MAX_W);
  if (pos < 0) return fail(1, "swa_decode_step: pos must be >= 0, got %d", pos);
  return hip_status(lz::launch_swa_decode(q, k_cache, v_cache, meta, n_meta, y, batch * heads,
                                          window, dim, pos, scale, heads / kv_heads,
                                          (hipStream_t)stream),
                    "swa_decode_step");
}

extern "C" size_t lz_swa_bwd_workspace_bytes(int batch, int heads, int length, int dim,
                                             int n_meta) {
  (void)dim;
  if (batch <= 0 || heads <= 0 || length <= 0 || n_meta < 0) return 0;
  const size_t bh = (size_t)batch * heads;
  return (bh * length + bh * lz::swa_row_blocks(length) * n_meta) * sizeof(float);
}

extern "C" int lz_swa_bwd(const void* q, const void* k, const void* v, const float* meta,
                          int n_meta, const float* lse, const void* dy, void* dq, void* dk,
                          void* dv, float* dmeta, int grad_bf16, int batch, int heads,
                          int kv_heads, int length, int dim, int window, float scale,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_swa(q, k, v, meta, n_meta, batch, heads, length, dim, window)) return rc;
  if (int rc = check_kv_heads("swa_bwd", heads, kv_heads)) return rc;
  if (!lse || !dy || !dq || !dk || !dv) return fail(1, "swa_bwd: null pointer");
  if (n_meta > 0 && !dmeta) return fail(1, "swa_bwd: null dmeta pointer");
  const size_t need = lz_swa_bwd_workspace_bytes(batch, heads, length, dim, n_meta);
  if (!workspace || workspace_bytes < need)
    return fail(1, "swa_bwd: workspace of %zu bytes given, %zu needed", workspace_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  float* delta = (float*)workspace;
  float* part = delta + (size_t)batch * heads * length;
  return hip_status(lz::launch_swa_bwd(q, k, v, meta, n_meta, lse, dy, dq, dk, dv,
                                       grad_bf16 != 0, delta, part, dmeta, batch * heads, length,
                                       dim, window, scale, heads / kv_heads, st),
                    "swa_bwd");
}

// ---------------------------------------------------------------------------
// layer prologue / epilogue
// ---------------------------------------------------------------------------
static int check_layer(int batch, int length, int heads, int kv_heads, int head_dim,
                       int feature_dim, bool bf16_in) {
  if (batch <= 0 || length <= 0 || heads <= 0 || kv_heads <= 0)
    return fail(1, "layer: sizes must be positive (B=%d L=%d heads=%d kv_heads=%d)", batch,
                length, heads, kv_heads);
  if (heads % kv_heads)
    return fail(1, "layer: heads (%d) must be a multiple of kv_heads (%d)", heads, kv_heads);
  if ((long long)batch * length * heads > (1LL << 31) - (1LL << 20))
    return fail(1, "layer: B*L*heads = %lld rows exceeds the 2^31 - 2^20 row limit",
                (long long)batch * length * heads);
  if (!lz::prologue_dims_supported(head_dim, feature_dim, bf16_in))
    return fail(1, "layer: unsupported head_dim %d / feature_dim %d (head_dim 32, 64 or 128; "
                   "feature_dim a multiple of 4 up to 128, up to 64 with head_dim 128 and "
                   "fp32 inputs)",
                head_dim, feature_dim);
  return 0;
}

extern "C" int lz_layer_prologue_fwd(const void* q, const void* k, const void* v, const void* wq,
                                     const void* wk, const void* cos, const void* sin,
                                     int cos_batched, void* fq, void* fk, void* qr, void* kr,
                                     void* v_out, int dtype_bf16, int batch, int length,
                                     int heads, int kv_heads, int head_dim, int feature_dim,
                                     void* stream) {
  if (int rc = check_layer(batch, length, heads, kv_heads, head_dim, feature_dim,
                             dtype_bf16 != 0))
    return rc;
  if (!q || !k || !v || !wq || !wk || !cos || !sin)
    return fail(1, "layer_prologue_fwd: null input pointer");
  if (!fk || !qr || !kr || !v_out) return fail(1, "layer_prologue_fwd: null output pointer");
  return hip_status(lz::launch_prologue_fwd(q, k, v, wq, wk, cos, sin, fq, fk, qr, kr, v_out,
                                            dtype_bf16 != 0, batch, length, heads, kv_heads,
                                            head_dim, feature_dim, cos_batched ? length : 0,
                                            (hipStream_t)stream),
                    "layer_prologue_fwd");
}

extern "C" size_t lz_layer_prologue_bwd_workspace_bytes(int batch, int length, int heads,
                                                        int kv_heads, int head_dim,
                                                        int feature_dim) {
  if (batch <= 0 || length <= 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads ||
      !lz::prologue_dims_supported(head_dim, feature_dim, true))
    return 0;
  return lz::prologue_bwd_workspace(batch, length, heads, kv_heads, head_dim, feature_dim);
}

extern "C" int lz_layer_prologue_bwd(const void* q, const void* k, const void* wq, const void* wk,
                                     const void* cos, const void* sin, int cos_batched,
                                     const void* dfq, const void* dfk, const void* dqr,
                                     const void* dkr, const void* dv, const void* dv2,
                                     void* dq, void* dk, void* dv_out, float* dwq, float* dwk,
                                     int dtype_bf16,
                                     int batch, int length, int heads, int kv_heads,
                                     int head_dim, int feature_dim, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  if (int rc = check_layer(batch, length, heads, kv_heads, head_dim, feature_dim,
                             dtype_bf16 != 0))
    return rc;
  if (!q || !k || !wq || !wk || !cos || !sin || !dfq || !dfk || !dqr || !dkr || !dv)
    return fail(1, "layer_prologue_bwd: null input pointer");
  if (!dq || !dk || !dv_out || !dwq || !dwk)
    return fail(1, "layer_prologue_bwd: null output pointer");
  const size_t need = lz_layer_prologue_bwd_workspace_bytes(batch, length, heads, kv_heads,
                                                            head_dim, feature_dim);
  if (!workspace || workspace_bytes < need)
    return fail(1, "layer_prologue_bwd: workspace of %zu bytes given, %zu needed",
                workspace_bytes, need);
  return hip_status(lz::launch_prologue_bwd(q, k, wq, wk, cos, sin, dfq, dfk, dqr, dkr, dv, dv2,
                                            dq, dk, dv_out, dwq, dwk, dtype_bf16 != 0, batch, length,
                                            heads, kv_heads, head_dim, feature_dim,
                                            cos_batched ? length : 0, (float*)workspace,
                                            (hipStream_t)stream),
                    "layer_prologue_bwd");
}

static int check_combine(int batch, int heads, int length, int head_dim) {
  if (batch <= 0 || heads <= 0 || length <= 0 || head_dim <= 0)
    return fail(1, "layer_combine: sizes must be positive (B=%d heads=%d L=%d hd=%d)", batch,
                heads, length, head_dim);
  if (head_dim % 8) return fail(1, "layer_combine: head_dim %d is not a multiple of 8", head_dim);
  return 0;
}

extern "C" int lz_layer_combine_fwd(const void* y_gla, const void* y_swa, const float* alpha,
                                    void* out, int out_bf16, int batch, int heads, int length,
                                    int head_dim, void* stream) {
  if (int rc = check_combine(batch, heads, length, head_dim)) return rc;
  if (!y_gla || !y_swa || !alpha || !out) return fail(1, "layer_combine_fwd: null pointer");
  return hip_status(lz::launch_combine_fwd(y_gla, y_swa, alpha, out, out_bf16 != 0, batch, heads,
                                           length, head_dim, (hipStream_t)stream),
                    "layer_combine_fwd");
}

extern "C" size_t lz_layer_combine_bwd_workspace_bytes(void) {
  return lz::combine_bwd_workspace();
}

extern "C" int lz_layer_combine_bwd(const void* dout, const void* y_swa, const float* alpha,
                                    void* dy_gla, void* dy_swa, float* dalpha, int out_bf16,
                                    int batch, int heads, int length, int head_dim,
                                    void* workspace, size_t workspace_bytes, void* stream) {
  if (int rc = check_combine(batch, heads, length, head_dim)) return rc;
  if (!dout || !y_swa || !alpha || !dy_gla || !dy_swa || !dalpha)
    return fail(1, "layer_combine_bwd: null pointer");
  if (!workspace || workspace_bytes < lz::combine_bwd_workspace())
    return fail(1, "layer_combine_bwd: workspace of %zu bytes given, %zu needed",
                workspace_bytes, lz::combine_bwd_workspace());
  return hip_status(lz::launch_combine_bwd(dout, y_swa, alpha, dy_gla, dy_swa, dalpha,
                                           out_bf16 != 0, batch, heads, length, head_dim,
                                           (float*)workspace, (hipStream_t)stream),
                    "layer_combine_bwd");
}
