// Pieces shared by the GLA forward and backward kernels: chunk staging,
// the chunk-local gate scan, segment bookkeeping.
#pragma once
#include <type_traits>

#include "common.hpp"

namespace lz {

constexpr int GLA_C = 64;            // chunk length (tokens)
// (b, h, segment) workgroups wanted per launch at F <= 128: two per CU of
// the current device (512 on a whole MI355X)
inline int gla_target_wg() { return 2 * device_geom().cus; }

// compile-time register-set selectors of the double-buffered chunk prefetch
constexpr std::integral_constant<int, 0> SET0{};
constexpr std::integral_constant<int, 1> SET1{};

int gla_padded_dim(int n);
bool gla_dims_supported(int F, int D);

// Tiles of the (F, D) problem that the native walks take (gla_tiled.hip):
// nF feature tiles of Ft (the last one the rest), nD value tiles of Dt.
struct GlaTiles {
  int nF, Ft, nD, Dt;
  bool native() const { return nF == 1 && nD == 1; }
};
GlaTiles gla_tiles(int F, int D);

// The native walks (F, D within gla_dims_supported).  raw_den: see
// gla_fwd_kernel's RAW; ext_den / ext_delta: see gla_bwd_dq_kernel's EXT.
size_t gla_fwd_workspace(int B, int H, int L, int F, int D);
size_t gla_bwd_workspace(int B, int H, int L, int F, int D, int gate);
hipError_t launch_gla_fwd(const void* fq, const void* fk, const void* v, const float* lg, void* y,
                          int B, int H, int L, int F, int D, int gate, int KG, float* ws,
                          float* final_state, float* raw_den, hipStream_t st);
hipError_t launch_gla_bwd(const void* fq, const void* fk, const void* v, const float* lg,
                          const void* dy, void* dfq, void* dfk, void* dv, float* dlg,
                          bool grad_bf16, int B, int H, int L, int F, int D, int gate,
                          int KG, const float* fwd_ws, float* ws, const float* ext_den,
                          const float* ext_delta, hipStream_t st);
// Any F and D: the native walks, or tiles of them (gla_tiled.hip).
size_t gla_fwd_workspace_any(int B, int H, int L, int F, int D);
size_t gla_bwd_workspace_any(int B, int H, int L, int F, int D, int gate);
hipError_t launch_gla_fwd_any(const void* fq, const void* fk, const void* v, const float* lg,
                              void* y, int B, int H, int L, int F, int D, int gate,
                              int KG, void* ws, hipStream_t st);
hipError_t launch_gla_bwd_any(const void* fq, const void* fk, const void* v, const float* lg,
                              const void* dy, void* dfq, void* dfk, void* dv, float* dlg,
                              bool grad_bf16, int B, int H, int L, int F, int D,
                              int gate, int KG, const float* fwd_ws, void* ws,
                              hipStream_t st);
// Sets, on the current device, the LDS limit of every kernel launch_gla_fwd
// (without raw_den) and launch_gla_fwd_states can launch.
hipError_t gla_fwd_prepare();
void gla_segments(int BH, int L, int F, int* G, int* cps);
int gla_walk_segments(int BH, int G, int F);
size_t gla_segment_floats(int BH, int G, int F, int D);

// Rows [t0, t0+64) of a [L x ncols] bf16 matrix into registers, 16 bytes per
// load: thread slot idx = tid + 256 i covers row idx / (KP/8), columns
// 8 * (idx % (KP/8)) .. +8.  Zero outside the matrix.
template <int KP, int N, int AUX = 0>
__device__ __forceinline__ void load_chunk(uint4 (&reg)[N], const bf16* __restrict__ base, int t0,
                                           int L, int ncols, bool vec) {
  load_items<KP, 256, N, 256 * N, AUX>(reg, base, t0, L, ncols, vec);
}

template <int KP, int N>
__device__ __forceinline__ void store_chunk(const uint4 (&reg)[N], bf16* tile, int pitch) {
  constexpr int K8 = KP / 8;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int idx = threadIdx.x + 256 * i;
    *reinterpret_cast<uint4*>(tile + (idx / K8) * pitch + (idx % K8) * 8) = reg[i];
  }
}

// Row-scaled copy of a [64 x KP] row-major bf16 tile, bf16(x[t][c] * scale[t]),
// spread over the 256 threads as 16-byte items: item i of a thread covers row
// tid / (KP/8) + (2048/KP) i, columns 8 (tid % (KP/8)) .. +8 (KP/32 items).
// The thread also writes the sums over its rows of the rounded values, per
// column, to part[(tid / (KP/8)) * KP + column]: 2048/KP partial sums per
// column (part holds 2048 floats), which a later pass adds up.
template <int KP>
struct RowItems {
  static constexpr int K8 = KP / 8;
  static constexpr int N = KP / 32;          // items per thread
  static constexpr int RSTRIDE = 256 / K8;   // rows between a thread's items
  static constexpr int PARTS = 256 / K8;     // partial sums per column
};

template <int KP>
__device__ __forceinline__ void scale_rows(const bf16* tile, int pitch, const float* scale,
                                           uint4 (&out)[RowItems<KP>::N], float* part) {
  using R = RowItems<KP>;
  const int cg = threadIdx.x % R::K8, r0 = threadIdx.x / R::K8;
  float sum[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sum[e] = 0.f;
#pragma unroll
  for (int i = 0; i < R::N; ++i) {
    const int t = r0 + R::RSTRIDE * i;
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(tile + t * pitch + 8 * cg);
    const float s = scale[t];
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = to_bf16(to_f32(x[e]) * s);
      sum[e] += to_f32(o[e]);
    }
    out[i] = __builtin_bit_cast(uint4, o);
  }
  float* dst = part + r0 * KP + 8 * cg;
  *reinterpret_cast<f32x4*>(dst) = f32x4{sum[0], sum[1], sum[2], sum[3]};
  *reinterpret_cast<f32x4*>(dst + 4) = f32x4{sum[4], sum[5], sum[6], sum[7]};
}

template <int KP>
__device__ __forceinline__ void store_rows(const uint4 (&in)[RowItems<KP>::N], bf16* tile,
                                           int pitch) {
  using R = RowItems<KP>;
  const int cg = threadIdx.x % R::K8, r0 = threadIdx.x / R::K8;
#pragma unroll
  for (int i = 0; i < R::N; ++i)
    *reinterpret_cast<uint4*>(tile + (r0 + R::RSTRIDE * i) * pitch + 8 * cg) = in[i];
}

// scale_rows for 256 threads numbered t (the upper half of an eight-wave
// workgroup, t = tid - 256), and its store_rows
template <int KP>
__device__ __forceinline__ void scale_rows_t(const bf16* tile, int pitch, const float* scale,
                                             uint4 (&out)[RowItems<KP>::N], float* part, int t) {
  using R = RowItems<KP>;
  const int cg = t % R::K8, r0 = t / R::K8;
  float sum[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sum[e] = 0.f;
#pragma unroll
  for (int i = 0; i < R::N; ++i) {
    const int row = r0 + R::RSTRIDE * i;
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(tile + row * pitch + 8 * cg);
    const float s = scale[row];
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = to_bf16(to_f32(x[e]) * s);
      sum[e] += to_f32(o[e]);
    }
    out[i] = __builtin_bit_cast(uint4, o);
  }
  float* dst = part + r0 * KP + 8 * cg;
  *reinterpret_cast<f32x4*>(dst) = f32x4{sum[0], sum[1], sum[2], sum[3]};
  *reinterpret_cast<f32x4*>(dst + 4) = f32x4{sum[4], sum[5], sum[6], sum[7]};
}

template <int KP>
__device__ __forceinline__ void store_rows_t(const uint4 (&in)[RowItems<KP>::N], bf16* tile,
                                             int pitch, int t) {
  using R = RowItems<KP>;
  const int cg = t % R::K8, r0 = t / R::K8;
#pragma unroll
  for (int i = 0; i < R::N; ++i)
    *reinterpret_cast<uint4*>(tile + (r0 + R::RSTRIDE * i) * pitch + 8 * cg) = in[i];
}

// The column sums of scale_rows alone, for a tile that is not rewritten:
// thread tid sums x[t][c] * scale[t] (rounded to bf16 first if ROUND, as
// scale_rows' values are) over its rows t = tid / (KP/8) + (2048/KP) i and its
// 8 columns c, into the same part[] layout (16-byte reads).
template <int KP, bool ROUND = true>
__device__ __forceinline__ void column_sums(const bf16* tile, int pitch, const float* scale,
                                            float* part) {
  using R = RowItems<KP>;
  const int cg = threadIdx.x % R::K8, r0 = threadIdx.x / R::K8;
  float sum[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) sum[e] = 0.f;
#pragma unroll
  for (int i = 0; i < R::N; ++i) {
    const int t = r0 + R::RSTRIDE * i;
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(tile + t * pitch + 8 * cg);
    const float s = scale[t];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = to_f32(x[e]) * s;
      sum[e] += ROUND ? to_f32(to_bf16(p)) : p;
    }
  }
  float* dst = part + r0 * KP + 8 * cg;
  *reinterpret_cast<f32x4*>(dst) = f32x4{sum[0], sum[1], sum[2], sum[3]};
  *reinterpret_cast<f32x4*>(dst + 4) = f32x4{sum[4], sum[5], sum[6], sum[7]};
}

// column c of the partial sums written by scale_rows (threads with tid < KP)
template <int KP>
__device__ __forceinline__ float sum_parts(const float* part, int c) {
  float s = 0.f;
#pragma unroll 8
  for (int p = 0; p < RowItems<KP>::PARTS; ++p) s += part[p * KP + c];
  return s;
}

// x + (x of the lane DPP control CTRL names); lanes with no source and lanes
// of rows outside ROW_MASK add 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_add(float x) {
  const int y = __builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xf, false);
  return x + __int_as_float(y);
}

// Inclusive prefix sum over the 64 lanes of a wave: Hillis-Steele steps of 1,
// 2, 4, 8 inside each 16-lane row (DPP row_shr), then the row totals carried
// up by row_bcast:15 (row r's last lane into row r + 1, rows 1 and 3) and
// row_bcast:31 (lane 31 into rows 2 and 3).  DPP moves need no LDS round
// trip, unlike the ds_bpermute behind __shfl_up.
__device__ __forceinline__ float wave_prefix_sum(float x) {
  x = dpp_add<0x111, 0xf>(x);   // row_shr:1
  x = dpp_add<0x112, 0xf>(x);   // row_shr:2
  x = dpp_add<0x114, 0xf>(x);   // row_shr:4
  x = dpp_add<0x118, 0xf>(x);   // row_shr:8
  x = dpp_add<0x142, 0xa>(x);   // row_bcast:15
  x = dpp_add<0x143, 0xc>(x);   // row_bcast:31
  return x;
}

// Inclusive suffix sum over the 64 lanes of a wave (lane l gets the sum of
// lanes l .. 63): the prefix sum of the lane-reversed values, reversed back.
__device__ __forceinline__ float wave_suffix_sum(float x, int lane) {
  x = __shfl(x, 63 - lane);
  x = wave_prefix_sum(x);
  return __shfl(x, 63 - lane);
}


// logsigmoid(z) = min(z, 0) - log(1 + e^{-|z|}), no overflow for any z, from
// the hardware exp2 and log2 (a few instructions: it sits in the walks' gate
// scan, where log1pf's longer sequence slowed the 256-register forward walk by
// 6 %).  For |z| > 17, 1 + e^{-|z|} rounds to 1 and the result to min(z, 0):
// an absolute error under 5e-8 in a log-gate.
__device__ __forceinline__ float log_sigmoid(float z) {
  return fminf(z, 0.f) - flog(1.f + fexp(-fabsf(z)));
}

// d logsigmoid(z) / dz = sigmoid(-z) = 1 / (1 + e^z) (0 when e^z overflows)
__device__ __forceinline__ float sigmoid_neg(float z) { return 1.f / (1.f + fexp(z)); }

// log_gamma from a gate buffer value of a token inside L, in mode `gate`
__device__ __forceinline__ float gate_log(float g, int gate) {
  return (gate & GATE_LOGIT) ? log_sigmoid(g) : g;
}

// Chunk-local inclusive scan of the gate by one wave (lane = token): lg,
// e^{lg}, e^{lg_end - lg}, and e^{lg_end}, lg_end in r[0], r[1].  g is the
// lane's raw gate value (0 past L); in GATE_LOGIT mode it is the logit,
// turned into logsigmoid(g) here (where it is used, so a prefetched gate is
// not waited for at its load) and 0 for a token past L (`valid` false).
__device__ __forceinline__ void gate_scan(float g, int lane, float* lgs, float* qs, float* ks,
                                          float* r, int gate, bool valid) {
  if (__builtin_expect(gate & GATE_LOGIT, 0)) g = valid ? log_sigmoid(g) : 0.f;
  g = wave_prefix_sum(g);
  const float end = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(g), 63));
  lgs[lane] = g;
  qs[lane] = fexp(g);
  ks[lane] = fexp(end - g);
  if (lane == 0) {
    r[0] = fexp(end);
    r[1] = end;
  }
}

// Causal decay of one 32 x 32 score tile s^T (keys kt*32 .. +32 x the query
// qi of this lane's column): p = bf16(s e^{lg_q - lg_k}) where k <= q, else
// 0, packed as the two MFMA fragments of the lane's 16 registers.  Returns
// the lane's partial sum of the rounded p (its half of the tile's rows).  The
// keys of registers 4 g .. 4 g + 3 are consecutive, so their gate logs come
// in as four 16-byte LDS reads, and the mask is a select: written per
// register with the key's log read under the condition, the compiler turned
// each of the 16 into a branch around its own LDS round trip.
__device__ __forceinline__ float decay_tile(const f32x16& s, const float* lgs, int kt, int qi,
                                            int h, bf16x8 (&p)[2]) {
  const float lgq = lgs[qi];
  float rsum = 0.f;
#pragma unroll
  for (int g4 = 0; g4 < 4; ++g4) {
    const int k0 = kt * 32 + 8 * g4 + 4 * h;   // keys of registers 4 g4 .. +4
    const f32x4 lk = *reinterpret_cast<const f32x4*>(lgs + k0);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int r = 4 * g4 + e;
      const float dec = k0 + e <= qi ? fexp(lgq - lk[e]) : 0.f;
      const bf16 pb = to_bf16(s[r] * dec);
      p[r >> 3][r & 7] = pb;
      rsum += to_f32(pb);
    }
  }
  return rsum;
}

// raw gate value of token t of a gate row of length L, 0 past its end (the
// mode is applied where it is used: gate_scan)
__device__ __forceinline__ float gate_at(const float* __restrict__ lgb, int t, int L) {
  return bload_f32(make_rsrc(lgb, (size_t)L * 4), (uint32_t)t * 4u);
}

// Which 32-wide tiles of a dimension with NT32 tiles a wave owns (i <
// TILES), and which 32-token halves of the chunk it pairs each with (j <
// HALVES).  Every (tile, half) pair has exactly one owner; with fewer than 4
// tiles a tile is owned by two waves (one per half), which then both carry
// that tile's state; `primary` marks the one of them that publishes it.
template <int NT32>
struct Roles {
  static constexpr int TILES = NT32 >= 4 ? NT32 / 4 : 1;
  static constexpr int HALVES = NT32 >= 4 ? 2 : 1;
  __device__ static bool active(int wave) { return NT32 >= 2 || wave < 2; }
  __device__ static bool primary(int wave) {
    return NT32 >= 4 || (NT32 == 2 ? wave < 2 : wave == 0);
  }
  __device__ static int tile(int wave, int i) {
    return NT32 >= 4 ? wave + 4 * i : (NT32 == 2 ? (wave & 1) : 0);
  }
  __device__ static int half(int wave, int j) {
    return NT32 >= 4 ? j : (NT32 == 2 ? (wave >> 1) : (wave & 1));
  }
};

// Block order of the walks.  With kv heads shared by KG > 1 query heads, the
// walks of one kv head's query heads read the same fk and v tiles: they are
// placed on one XCD (one L2) by xcd_block, the grid padded to a multiple of
// the XCD count.  With KG = 1 the launch order is kept (the grouped order
// measured slower there).
struct WalkGrid {
  int grid, per, nx, nblk;   // per = 0: launch order; nx = the device's XCDs
};
inline WalkGrid walk_grid(int nblk, int KG) {
  if (KG <= 1) return WalkGrid{nblk, 0, device_geom().xcds, nblk};
  const int nx = device_geom().xcds;
  const int grid = xcd_grid(nblk, nx);
  return WalkGrid{grid, grid / nx, nx, nblk};
}

// Logical block of this walk workgroup; false for the padding blocks of a
// grouped grid (the whole workgroup returns before any barrier).
// rev: the workgroups of each XCD (workgroup i runs on XCD i % nx) take that
// XCD's blocks in reverse launch order, each block kept on its XCD.  A walk
// launched in more than one round of workgroups after a walk over the same
// rows in launch order then starts on the rows that walk read last, which the
// memory-side cache (and for the last chunks the XCD's L2) still holds.
__device__ __forceinline__ bool walk_block(int xper, int nx, int nblk, int& blk,
                                           bool rev = false) {
  int b = (int)blockIdx.x;
  if (rev) {
    const int full = (int)gridDim.x - (int)gridDim.x % nx;
    if (b < full) b = full - nx - (b - b % nx) + b % nx;
  }
  blk = xper ? xcd_block(b, xper, nx) : b;
  return blk < nblk;
}

// Forward segment records belong to kv heads when the gate is per token: the
// KG query heads of a kv head then see the same fk, v and gate, hence the same
// segment states, which the state pass computes once.  The record of query
// head bh:
__host__ __device__ inline int seg_owner(int bh, int KG, int gate) {
  return (gate & GATE_PER_HEAD) ? bh : bh / KG;
}
// The same inside a walk, marked wave-uniform: used as written above in the
// record pointer, it led the compiler to take the walks' chunk buffer
// resources for divergent and to wrap every chunk load in a readfirstlane
// loop.
__device__ __forceinline__ int seg_owner_uniform(int bh, int KG, int gate) {
  return __builtin_amdgcn_readfirstlane(seg_owner(bh, KG, gate));
}

// Per-(b, h, segment) state record: S [FP][DP] fp32, then z [FP].
template <int FP, int DP>
struct SegRec {
  static constexpr int SIZE = FP * DP + FP;
};

// Records one pass of fold_records loads together: VREGS / 4 16-byte loads
// in flight per thread, at least one record and at most 8.
__host__ __device__ constexpr int fold_batch(int T, int REC, int VREGS) {
  return (VREGS / 4 / ((REC / 4 + T - 1) / T)) < 1 ? 1
         : (VREGS / 4 / ((REC / 4 + T - 1) / T)) > 8 ? 8
                                                      : VREGS / 4 / ((REC / 4 + T - 1) / T);
}

// The state entering a segment, formed inside a walk from the local records
// of the segments on its left (forward: records first, first + 1, ...) or on
// its right (reverse: first, first - 1, ...), n records, in the order and with
// the arithmetic of gla_segment_scan_kernel: carry = e^{lam_g} carry + R_g,
// one fused multiply-add per element.  So the state has the bits the scan
// would have written.  The T threads of the workgroup fold the REC floats of a
// record as 16-byte groups and write the result to out (LDS, 16-byte aligned),
// with VREGS registers of loads in flight per thread (the walk's own registers
// bound it: its chunk loads are in flight meanwhile).
template <int T, int REC, int VREGS>
__device__ __forceinline__ void fold_records(float* __restrict__ out,
                                             const float* __restrict__ base,
                                             const float* __restrict__ lam, int first, int step,
                                             int n) {
  static_assert(REC % 4 == 0, "records are whole 16-byte groups");
  constexpr int N4 = REC / 4, NG = (N4 + T - 1) / T, FB = fold_batch(T, REC, VREGS);
  const int tid = threadIdx.x;
  f32x4 carry[NG];
#pragma unroll
  for (int k = 0; k < NG; ++k) carry[k] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int g0 = 0; g0 < n; g0 += FB) {
    f32x4 d[FB][NG];
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      const bool ok = g0 + b < n;   // wave-uniform
      const float* rec = base + (size_t)(first + step * (g0 + b)) * REC;
#pragma unroll
      for (int k = 0; k < NG; ++k) {
        const int i = tid + T * k;
        d[b][k] = ok && (N4 % T == 0 || i < N4) ? *reinterpret_cast<const f32x4*>(rec + 4 * i)
                                                : f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
#pragma unroll
    for (int b = 0; b < FB; ++b) {
      if (g0 + b < n) {
        const float w = fexp(lam[first + step * (g0 + b)]);
#pragma unroll
        for (int k = 0; k < NG; ++k)
#pragma unroll
          for (int c = 0; c < 4; ++c) carry[k][c] = __builtin_fmaf(w, carry[k][c], d[b][k][c]);
      }
    }
  }
#pragma unroll
  for (int k = 0; k < NG; ++k) {
    const int i = tid + T * k;
    if (N4 % T == 0 || i < N4) *reinterpret_cast<f32x4*>(out + 4 * i) = carry[k];
  }
}

// Whether the walks fold the segment records themselves (no scan launch):
// for at most 4 segments per row, in the walks that have a folding variant
// (whole 16-byte rows, records of at least 128 x 64 floats).  Measured: with
// 4 segments (F = D = 128, B = 4, L = 2048) and 3 (F = 256, D = 64, the
// config-5 layer) the fold took 6-11 us off a fwd+bwd; with 16 (F = D = 64,
// B = 1, L = 2048) its passes over 15 records of each walk cost more than
// the scan launch.  The state passes leave the records unscanned exactly
// when the walks that read them fold.
template <int FP, int DP, bool VEC>
constexpr bool gla_can_fold() {
  return VEC && FP * DP >= 128 * 64;
}
inline bool gla_fold_segments(int G) { return G > 1 && G <= 4; }

// Segment pass of the forward recurrence (gla_fwd.hip) and the scan over
// segments; used by the forward and by the backward's forward walk.
// fold: the walks fold the records (no scan).
hipError_t launch_gla_fwd_states(const void* fk, const void* v, const float* lg, float* seg_state,
                                 float* seg_logdecay, int BH, int H, int L, int F, int D,
                                 int gate, int G, int cps, int KG, bool fold, hipStream_t st);
hipError_t launch_gla_segment_scan(float* seg_state, const float* seg_logdecay, int BH, int G,
                                   int rec, bool reverse, hipStream_t st);

}  // namespace lz
