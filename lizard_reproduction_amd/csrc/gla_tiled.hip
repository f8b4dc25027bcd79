// GLA at feature and value dims beyond the walks' own (F <= 256, D <= 128,
// D <= 64 when F > 128): the operator takes any F and D, as the reference's
// kernels do by looping over feature blocks (src/kernels/gla.py:74,154,171)
// and sizing their value block from D (gla.py:203-210).  Here the native
// walks run on tiles of the problem and their results are combined:
//
//   D tiles: y = N / den with N = sum_t w_it v_t column by column and den
//   independent of D, so each D tile of v gives exactly its columns of y.  In
//   the backward every gradient is linear in dy given den and delta =
//   sum_d dy y, and delta splits over D tiles (delta_t = sum_{d in t} dy y):
//   each tile's walk forms its own den (all of F) and delta_t, and dfq, dfk
//   and d log_gamma are the sums of the tiles' (in fp32), dv the tiles' columns.
//
//   F tiles (F > 256): the scores w_it = (fq_i . fk_t) decay_it, hence N and
//   den, are sums over feature tiles.  Each tile's walk writes its
//   unnormalised numerator and denominator (RAW), which are summed and
//   divided (a, the bf16 weights, is rounded per tile: the same bf16
//   tolerance, the same invariants -- constant v stays constant, L = 1
//   gives v).  The backward of tile f needs the whole den and delta
//   (dL/dN = dy / den, dL/dden = -delta / den): it recomputes N and den
//   through the RAW walks, forms delta_t for each D tile, and runs each
//   (F tile, D tile) walk with that den and delta (EXT).  dfq and dfk of
//   tile f are its columns, dv and d log_gamma sums over the tiles.
//
// Operand tiles are copied into contiguous workspace buffers (the walks read
// contiguous [rows, width] slabs); partial results are summed in fp32 in a
// fixed order (tiles in order, one launch each), so results stay
// deterministic.
#include <algorithm>

#include "gla_common.hpp"

namespace lz {

namespace {

int round8(int x) { return (x + 7) / 8 * 8; }

}  // namespace

GlaTiles gla_tiles(int F, int D) {
  if (gla_dims_supported(F, D)) return GlaTiles{1, F, 1, D};
  int nF = 1, Ft = F;
  if (F > 256) {   // F tiles of at most 256 features (128 when D needs tiles of 128)
    const int fmax = D <= 64 ? 256 : 128;
    nF = (F + fmax - 1) / fmax;
    Ft = round8((F + nF - 1) / nF);
    nF = (F + Ft - 1) / Ft;
  }
  const int dmax = gla_padded_dim(Ft) > 128 ? 64 : 128;
  int nD = (D + dmax - 1) / dmax;
  const int Dt = round8((D + nD - 1) / nD);
  nD = (D + Dt - 1) / Dt;
  return GlaTiles{nF, Ft, nD, Dt};
}

namespace {

// ---------------------------------------------------------------------------
// helper kernels: column blocks, sums, the combine of split-F partials
// ---------------------------------------------------------------------------
// dst[r][dc0 + c] (+)= src[r][sc0 + c] for r < rows, c < w (row pitches pd, ps)
template <typename DstT, typename SrcT, bool ADD>
__global__ __launch_bounds__(256) void gla_block_kernel(DstT* __restrict__ dst, int pd, int dc0,
                                                        const SrcT* __restrict__ src, int ps,
                                                        int sc0, int w, size_t rows) {
  const size_t n = rows * (size_t)w;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const size_t r = i / w, c = i % w;
    float val = static_cast<float>(src[r * ps + sc0 + c]);
    DstT* d = dst + r * pd + dc0 + c;
    if constexpr (ADD) val += static_cast<float>(*d);
    *d = static_cast<DstT>(val);
  }
}

// y[r][c] = bf16(num[r][c] / max(den[r], FLT_MIN))
__global__ __launch_bounds__(256) void gla_combine_kernel(bf16* __restrict__ y,
                                                          const float* __restrict__ num,
                                                          const float* __restrict__ den, int D,
                                                          size_t rows) {
  const size_t n = rows * (size_t)D;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    y[i] = to_bf16(num[i] / fmaxf(den[i / D], TINY));
}

// delta[r] = sum_{c0 <= c < c0 + w} dy[r][c] * num[r][c] / max(den[r], FLT_MIN),
// one wave per row, the columns summed in a fixed order
__global__ __launch_bounds__(256) void gla_delta_kernel(float* __restrict__ delta,
                                                        const bf16* __restrict__ dy,
                                                        const float* __restrict__ num,
                                                        const float* __restrict__ den, int D,
                                                        int c0, int w, size_t rows) {
  const int lane = threadIdx.x & 63;
  for (size_t r = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6); r < rows;
       r += (size_t)gridDim.x * 4) {
    float s = 0.f;
    for (int c = lane; c < w; c += 64)
      s += to_f32(dy[r * D + c0 + c]) * num[r * D + c0 + c];
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) delta[r] = s / fmaxf(den[r], TINY);
  }
}

unsigned grid_for(size_t n) {
  const size_t g = (n + 255) / 256;
  return (unsigned)(g < 8192 ? (g ? g : 1) : 8192);
}

template <typename DstT, typename SrcT, bool ADD>
hipError_t block_op(DstT* dst, int pd, int dc0, const SrcT* src, int ps, int sc0, int w,
                    size_t rows, hipStream_t st) {
  hipLaunchKernelGGL((gla_block_kernel<DstT, SrcT, ADD>), dim3(grid_for(rows * w)), dim3(256),
                     0, st, dst, pd, dc0, src, ps, sc0, w, rows);
  return hipGetLastError();
}

// `first`: assign, else add
hipError_t put_f32(float* dst, int pd, int dc0, const float* src, int ps, int sc0, int w,
                   size_t rows, bool first, hipStream_t st) {
  return first ? block_op<float, float, false>(dst, pd, dc0, src, ps, sc0, w, rows, st)
               : block_op<float, float, true>(dst, pd, dc0, src, ps, sc0, w, rows, st);
}

hipError_t cast_out(void* dst, bool bf16_out, int pd, int dc0, const float* src, int ps, int w,
                    size_t rows, hipStream_t st) {
  return bf16_out ? block_op<bf16, float, false>((bf16*)dst, pd, dc0, src, ps, 0, w, rows, st)
                  : block_op<float, float, false>((float*)dst, pd, dc0, src, ps, 0, w, rows, st);
}

hipError_t copy_bf16(bf16* dst, int pd, int dc0, const bf16* src, int ps, int sc0, int w,
                     size_t rows, hipStream_t st) {
  return block_op<bf16, bf16, false>(dst, pd, dc0, src, ps, sc0, w, rows, st);
}

// A bump allocator over a caller's workspace (256-byte aligned pieces).
struct Carve {
  char* p;
  size_t used = 0;
  template <typename T>
  T* take(size_t n) {
    T* r = p ? reinterpret_cast<T*>(p + used) : nullptr;
    used += (n * sizeof(T) + 255) / 256 * 256;
    return r;
  }
};

int width_of(int i, int n, int t, int total) { return i + 1 < n ? t : total - (n - 1) * t; }

// The largest workspace a walk of any tile needs (the last tiles are narrower,
// and a narrower F tile may take another segment split).
template <typename Fn>
size_t max_over_tiles(const GlaTiles& t, int F, int D, Fn ws) {
  const int fl = width_of(t.nF - 1, t.nF, t.Ft, F), dl = width_of(t.nD - 1, t.nD, t.Dt, D);
  size_t m = ws(t.Ft, t.Dt);
  m = std::max(m, ws(fl, t.Dt));
  m = std::max(m, ws(t.Ft, dl));
  return std::max(m, ws(fl, dl));
}

// The buffers of the tiled forward (workspace `ws`, or sizing when null).
struct FwdBufs {
  bf16 *fqt, *fkt, *vt, *yt;
  float *numt, *dent, *num, *den;
  float* inner;
  size_t inner_bytes;
};

FwdBufs carve_fwd(Carve& c, const GlaTiles& t, int B, int H, int L, int F, int D) {
  const size_t BHL = (size_t)B * H * L;
  FwdBufs b{};
  b.inner_bytes = max_over_tiles(t, F, D, [&](int f, int d) {
    return gla_fwd_workspace(B, H, L, f, d);
  });
  if (t.nF == 1) {
    b.vt = c.take<bf16>(BHL * t.Dt);
    b.yt = c.take<bf16>(BHL * t.Dt);
  } else {
    b.fqt = c.take<bf16>(BHL * t.Ft);
    b.fkt = c.take<bf16>(BHL * t.Ft);
    if (t.nD > 1) b.vt = c.take<bf16>(BHL * t.Dt);
    b.numt = c.take<float>(BHL * t.Dt);
    b.dent = c.take<float>(BHL);
    b.num = c.take<float>(BHL * D);
    b.den = c.take<float>(BHL);
  }
  b.inner = c.take<float>((b.inner_bytes + 3) / 4);
  return b;
}

// The RAW walks over all (F tile, D tile) pairs: num [BH, L, D] and den [BH, L]
// of the whole feature dimension, summed over the F tiles in order.
hipError_t raw_forward(const GlaTiles& t, const FwdBufs& b, const void* fq, const void* fk,
                       const void* v, const float* lg, int B, int H, int L, int F, int D, int gph,
                       int KG, hipStream_t st) {
  const size_t BHL = (size_t)B * H * L, BHLk = BHL / KG;
  hipError_t e;
  for (int f = 0; f < t.nF; ++f) {
    const int fw = width_of(f, t.nF, t.Ft, F);
    if ((e = copy_bf16(b.fqt, fw, 0, (const bf16*)fq, F, f * t.Ft, fw, BHL, st))) return e;
    if ((e = copy_bf16(b.fkt, fw, 0, (const bf16*)fk, F, f * t.Ft, fw, BHLk, st))) return e;
    for (int d = 0; d < t.nD; ++d) {
      const int dw = width_of(d, t.nD, t.Dt, D);
      const bf16* vt = (const bf16*)v;
      if (t.nD > 1) {
        if ((e = copy_bf16(b.vt, dw, 0, (const bf16*)v, D, d * t.Dt, dw, BHLk, st))) return e;
        vt = b.vt;
      }
      if ((e = launch_gla_fwd(b.fqt, b.fkt, vt, lg, b.numt, B, H, L, fw, dw, gph, KG, b.inner,
                              nullptr, b.dent, st)))
        return e;
      if ((e = put_f32(b.num, D, d * t.Dt, b.numt, dw, 0, dw, BHL, f == 0, st))) return e;
      if (d == 0 && (e = put_f32(b.den, 1, 0, b.dent, 1, 0, 1, BHL, f == 0, st))) return e;
    }
  }
  return hipSuccess;
}

}  // namespace

size_t gla_fwd_workspace_any(int B, int H, int L, int F, int D) {
  const GlaTiles t = gla_tiles(F, D);
  if (t.native()) return gla_fwd_workspace(B, H, L, F, D);
  Carve c{nullptr};
  carve_fwd(c, t, B, H, L, F, D);
  return c.used;
}

hipError_t launch_gla_fwd_any(const void* fq, const void* fk, const void* v, const float* lg,
                              void* y, int B, int H, int L, int F, int D, int gph, int KG,
                              void* ws, hipStream_t st) {
  const GlaTiles t = gla_tiles(F, D);
  if (t.native())
    return launch_gla_fwd(fq, fk, v, lg, y, B, H, L, F, D, gph, KG, (float*)ws, nullptr, nullptr,
                          st);
  Carve c{(char*)ws};
  const FwdBufs b = carve_fwd(c, t, B, H, L, F, D);
  const size_t BHL = (size_t)B * H * L, BHLk = BHL / KG;
  hipError_t e;
  if (t.nF == 1) {   // D tiles of the native walk, each its own columns of y
    for (int d = 0; d < t.nD; ++d) {
      const int dw = width_of(d, t.nD, t.Dt, D);
      // every D tile reads fq and fk again: only the last may load them as
      // read no more (GATE_NO_REUSE)
      const int gd = d + 1 < t.nD ? gph & ~GATE_NO_REUSE : gph;
      if ((e = copy_bf16(b.vt, dw, 0, (const bf16*)v, D, d * t.Dt, dw, BHLk, st))) return e;
      if ((e = launch_gla_fwd(fq, fk, b.vt, lg, b.yt, B, H, L, F, dw, gd, KG, b.inner, nullptr,
                              nullptr, st)))
        return e;
      if ((e = copy_bf16((bf16*)y, D, d * t.Dt, b.yt, dw, 0, dw, BHL, st))) return e;
    }
    return hipSuccess;
  }
  if ((e = raw_forward(t, b, fq, fk, v, lg, B, H, L, F, D, gph, KG, st))) return e;
  hipLaunchKernelGGL(gla_combine_kernel, dim3(grid_for(BHL * D)), dim3(256), 0, st, (bf16*)y,
                     (const float*)b.num, (const float*)b.den, D, BHL);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
namespace {

struct BwdBufs {
  FwdBufs fwd;           // F split: the recomputed num and den
  bf16 *vt, *dyt;        // the D tile of v and dy
  float* delta;          // F split: [nD][BH L] delta of each D tile
  float *dfq_t, *dfk_t, *dv_t, *dlg_t;      // one walk's gradients (fp32)
  float *dfq_a, *dfk_a, *dv_a, *dlg_a;      // their sums (fp32)
  float* inner;
  size_t inner_bytes;
};

BwdBufs carve_bwd(Carve& c, const GlaTiles& t, int B, int H, int L, int F, int D, int gph) {
  const size_t BHL = (size_t)B * H * L, NG = (gph & GATE_PER_HEAD) ? BHL : (size_t)B * L;
  BwdBufs b{};
  if (t.nF > 1) b.fwd = carve_fwd(c, t, B, H, L, F, D);
  b.vt = c.take<bf16>(BHL * t.Dt);
  b.dyt = c.take<bf16>(BHL * t.Dt);
  if (t.nF > 1) b.delta = c.take<float>(BHL * t.nD);
  b.dfq_t = c.take<float>(BHL * t.Ft);
  b.dfk_t = c.take<float>(BHL * t.Ft);
  b.dv_t = c.take<float>(BHL * t.Dt);
  b.dlg_t = c.take<float>(NG);
  b.dfq_a = c.take<float>(BHL * F);
  b.dfk_a = c.take<float>(BHL * F);
  if (t.nF > 1) b.dv_a = c.take<float>(BHL * D);
  b.dlg_a = c.take<float>(NG);
  b.inner_bytes = max_over_tiles(t, F, D, [&](int f, int d) {
    return gla_bwd_workspace(B, H, L, f, d, gph);
  });
  b.inner = c.take<float>((b.inner_bytes + 3) / 4);
  return b;
}

}  // namespace

size_t gla_bwd_workspace_any(int B, int H, int L, int F, int D, int gph) {
  const GlaTiles t = gla_tiles(F, D);
  if (t.native()) return gla_bwd_workspace(B, H, L, F, D, gph);
  Carve c{nullptr};
  carve_bwd(c, t, B, H, L, F, D, gph);
  return c.used;
}

hipError_t launch_gla_bwd_any(const void* fq, const void* fk, const void* v, const float* lg,
                              const void* dy, void* dfq, void* dfk, void* dv, float* dlg,
                              bool grad_bf16, int B, int H, int L, int F, int D, int gph, int KG,
                              const float* fwd_ws, void* ws, hipStream_t st) {
  const GlaTiles t = gla_tiles(F, D);
  if (t.native())
    return launch_gla_bwd(fq, fk, v, lg, dy, dfq, dfk, dv, dlg, grad_bf16, B, H, L, F, D, gph,
                          KG, fwd_ws, (float*)ws, nullptr, nullptr, st);
  Carve c{(char*)ws};
  const BwdBufs b = carve_bwd(c, t, B, H, L, F, D, gph);
  const size_t BHL = (size_t)B * H * L, BHLk = BHL / KG, NG = (gph & GATE_PER_HEAD) ? BHL : (size_t)B * L;
  hipError_t e;
  if (t.nF > 1) {   // num, den of the whole feature dimension, then delta per D tile
    if ((e = raw_forward(t, b.fwd, fq, fk, v, lg, B, H, L, F, D, gph, KG, st))) return e;
    for (int d = 0; d < t.nD; ++d) {
      hipLaunchKernelGGL(gla_delta_kernel, dim3(grid_for(BHL * 64)), dim3(256), 0,
                         st, b.delta + (size_t)d * BHL, (const bf16*)dy,
                         (const float*)b.fwd.num, (const float*)b.fwd.den, D, d * t.Dt,
                         width_of(d, t.nD, t.Dt, D), BHL);
      if ((e = hipGetLastError())) return e;
    }
  }
  for (int f = 0; f < t.nF; ++f) {
    const int fw = width_of(f, t.nF, t.Ft, F);
    const bf16 *fqt = (const bf16*)fq, *fkt = (const bf16*)fk;
    if (t.nF > 1) {
      if ((e = copy_bf16(b.fwd.fqt, fw, 0, (const bf16*)fq, F, f * t.Ft, fw, BHL, st))) return e;
      if ((e = copy_bf16(b.fwd.fkt, fw, 0, (const bf16*)fk, F, f * t.Ft, fw, BHLk, st))) return e;
      fqt = b.fwd.fqt;
      fkt = b.fwd.fkt;
    }
    for (int d = 0; d < t.nD; ++d) {
      const int dw = width_of(d, t.nD, t.Dt, D);
      const bool first = f == 0 && d == 0;
      const bf16 *vt = (const bf16*)v, *dyt = (const bf16*)dy;
      if (t.nD > 1) {
        if ((e = copy_bf16(b.vt, dw, 0, (const bf16*)v, D, d * t.Dt, dw, BHLk, st))) return e;
        if ((e = copy_bf16(b.dyt, dw, 0, (const bf16*)dy, D, d * t.Dt, dw, BHL, st))) return e;
        vt = b.vt;
        dyt = b.dyt;
      }
      const float* eden = t.nF > 1 ? b.fwd.den : nullptr;
      const float* edel = t.nF > 1 ? b.delta + (size_t)d * BHL : nullptr;
      if ((e = launch_gla_bwd(fqt, fkt, vt, lg, dyt, b.dfq_t, b.dfk_t, b.dv_t, b.dlg_t, false, B,
                              H, L, fw, dw, gph, KG, nullptr, b.inner, eden, edel, st)))
        return e;
      // dfq, dfk: this F tile's columns, summed over the D tiles
      if ((e = put_f32(b.dfq_a, F, f * t.Ft, b.dfq_t, fw, 0, fw, BHL, d == 0, st))) return e;
      if ((e = put_f32(b.dfk_a, F, f * t.Ft, b.dfk_t, fw, 0, fw, BHL, d == 0, st))) return e;
      // dv: this D tile's columns, summed over the F tiles
      if (t.nF > 1) {
        if ((e = put_f32(b.dv_a, D, d * t.Dt, b.dv_t, dw, 0, dw, BHL, f == 0, st))) return e;
      } else if ((e = cast_out(dv, grad_bf16, D, d * t.Dt, b.dv_t, dw, dw, BHL, st))) {
        return e;
      }
      if ((e = put_f32(b.dlg_a, 1, 0, b.dlg_t, 1, 0, 1, NG, first, st))) return e;
    }
  }
  if ((e = cast_out(dfq, grad_bf16, F, 0, b.dfq_a, F, F, BHL, st))) return e;
  if ((e = cast_out(dfk, grad_bf16, F, 0, b.dfk_a, F, F, BHL, st))) return e;
  if (t.nF > 1 && (e = cast_out(dv, grad_bf16, D, 0, b.dv_a, D, D, BHL, st))) return e;
  return cast_out(dlg, false, 1, 0, b.dlg_a, 1, 1, NG, st);
}

}  // namespace lz
