// Prologue and epilogue of the LizardAttention layer (src/lizard_attention.py:
// 78-97): everything between the q/k/v projections and o_proj except the two
// attention branches.
//
// Prologue, per token row of the projections ([B, L, heads, hd] row-major,
// rows ordered (b, l, head)):
//   fq = [softmax(q Wq^T), softmax(-q Wq^T)]      (Hedgehog, :9-11, F = 2f)
//   qr = rope(q)                                  (rotate_half RoPE, :88)
//   fk, kr, v likewise from the kv heads
// all in fp32 from the inputs' values, written once as the bf16 operands of
// the GLA and SWA kernels: [B, H, L, .] for the query side, [B, Hkv, L, .]
// for the key side.  The reference's repeat_interleave of k and v to the
// H / Hkv query heads of a group (:73-76) is not materialised: the GLA and
// SWA kernels read a query head's k-side operands from its kv head.  x W^T is a bf16 MFMA product; fp32
// inputs are split into bf16 hi + lo parts and the three significant partial
// products summed (hi*hi + lo*hi + hi*lo), which keeps fp32-level accuracy.
//
// Backward (from bf16 gradients of the five outputs): the softmax Jacobians give dxw = p (dp - <p,dp>) - n (dn - <n,dn>)
// (p, n recomputed from x W^T), dq = dxw W + rope^T(dqr), and
// dW = sum over rows of dxw^T q, reduced deterministically: per-workgroup
// partial tiles in a workspace, then one fixed-order sum.
//
// Epilogue: out[b, l, h*hd + d] = y_gla + alpha * y_swa (the blend of :94-96
// and the transpose/flatten of :97), and its backward with d alpha summed
// deterministically.
#include <algorithm>

#include "common.hpp"

namespace lz {

constexpr int PRO_WAVES = 4;
constexpr int PRO_ROWS = 32;                      // rows per wave and block
constexpr int PRO_BLOCK = PRO_WAVES * PRO_ROWS;   // rows per workgroup iteration
constexpr int PRO_BWD_WG_PER_CU = 2;              // the most any backward instantiation asks for
constexpr int CMB_BLOCKS = 1024;                  // epilogue backward partial sums

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <typename T>
__device__ __forceinline__ void load8f(const T* __restrict__ p, float (&x)[8]) {
  if constexpr (sizeof(T) == 2) {
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = to_f32(v[e]);
  } else {
    const f32x4 a = *reinterpret_cast<const f32x4*>(p);
    const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  }
}

template <typename T>
__device__ __forceinline__ f32x4 load4f(const T* __restrict__ p) {
  if constexpr (sizeof(T) == 2) {
    const bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
    return f32x4{to_f32(v[0]), to_f32(v[1]), to_f32(v[2]), to_f32(v[3])};
  } else {
    return *reinterpret_cast<const f32x4*>(p);
  }
}

template <typename T>
__device__ __forceinline__ void store4v(T* __restrict__ p, const f32x4& x) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<bf16x4*>(p) =
        bf16x4{to_bf16(x[0]), to_bf16(x[1]), to_bf16(x[2]), to_bf16(x[3])};
  } else {
    *reinterpret_cast<f32x4*>(p) = x;
  }
}

// 8 elements of T at p as raw registers (16 bytes of bf16, 32 of fp32), to be
// converted by cvt8 later: a row's loads can then all issue before any use.
template <typename T>
struct Raw8 {
  uint4 r[sizeof(T) / 2];
};

template <typename T>
__device__ __forceinline__ Raw8<T> load8r(const T* __restrict__ p) {
  Raw8<T> o;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 2); ++i) o.r[i] = reinterpret_cast<const uint4*>(p)[i];
  return o;
}

template <typename T>
__device__ __forceinline__ void cvt8(const Raw8<T>& v, float (&x)[8]) {
  if constexpr (sizeof(T) == 2) {
    const bf16x8 b = __builtin_bit_cast(bf16x8, v.r[0]);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = to_f32(b[e]);
  } else {
    const f32x4 a = __builtin_bit_cast(f32x4, v.r[0]), b = __builtin_bit_cast(f32x4, v.r[1]);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[e] = a[e];
      x[4 + e] = b[e];
    }
  }
}

__device__ __forceinline__ bf16x8 to_bf8(const float (&x)[8]) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to_bf16(x[e]);
  return o;
}

// bf16(x - hi): the low part of a two-term bf16 split of fp32 values
__device__ __forceinline__ bf16x8 low8(const float (&x)[8], const bf16x8& hi) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to_bf16(x[e] - to_f32(hi[e]));
  return o;
}

// Registers 8*kb .. 8*kb+7 of an accumulator minus their bf16 rounding.
__device__ __forceinline__ bf16x8 acc_operand_lo(const f32x16& acc, int kb) {
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float x = acc[8 * kb + j];
    o[j] = to_bf16(x - to_f32(to_bf16(x)));
  }
  return o;
}

// Tile shapes: FT 32-feature tiles (f <= 32 FT), HT 32-wide head-dim tiles
// (hd = 32 HT); T is the element type of the projections, weights and RoPE
// tables (float or bf16).
template <typename T, int FT, int HT>
struct Pro {
  static constexpr int FP = 32 * FT, HP = 32 * HT, HK = HP / 16;
  static constexpr bool SPLIT = sizeof(T) == 4;
  static constexpr int PARTS = SPLIT ? 2 : 1;
  static constexpr int WP = lds_pitch(HP);      // W tile [FP][WP] (rows = features)
  static constexpr int W_ELEMS = FP * WP;
  static constexpr int SP = lds_pitch(FP);      // forward staging [32][SP] per wave
  static constexpr int FWD_LDS = (PARTS * W_ELEMS + PRO_WAVES * PRO_ROWS * SP) * 2;
  static_assert(FWD_LDS <= 160 * 1024, "LDS budget");
};

struct ProFwdArgs {
  const void *q, *k, *v, *wq, *wk, *cos, *sin;
  bf16 *fq, *fk, *qr, *kr, *vo;
  int B, L, H, Hkv, hd, f, cos_bstride, nq_wg;
};

struct ProBwdArgs {
  const void *q, *k, *wq, *wk, *cos, *sin;
  const bf16 *dfq, *dfk, *dqr, *dkr, *dv, *dv2;   // dv2 may be null
  void *dq, *dk, *dvo;
  float* part;
  int B, L, H, Hkv, hd, f, cos_bstride;
  int nbq, nbk;   // 128-row blocks of the q rows and of the kv rows
};

// W [f][hd] (type T) into LDS as bf16 hi (and lo) tiles [FP][WP], zero rows
// beyond f.
template <typename T, int FT, int HT>
__device__ void load_weight(const T* __restrict__ w, int f, bf16* hi, bf16* lo) {
  using C = Pro<T, FT, HT>;
  for (int i = threadIdx.x; i < C::FP * C::HP; i += blockDim.x) {
    const int r = i / C::HP, c = i % C::HP;
    const float x = r < f ? static_cast<float>(w[r * C::HP + c]) : 0.f;
    const bf16 h = to_bf16(x);
    hi[r * C::WP + c] = h;
    if constexpr (C::SPLIT) lo[r * C::WP + c] = to_bf16(x - to_f32(h));
  }
}

// Tile ft of x W^T for the 32 rows of a wave: features 32 ft + acc_row(r, h)
// (registers) of row lane % 32 (lanes).  The kernels recompute a tile in each
// pass that needs it rather than keep all of them live: the MFMA work is
// small next to the memory traffic, and the registers buy occupancy.
template <typename T, int FT, int HT>
__device__ __forceinline__ f32x16 project_tile(int ft, const bf16x8 (&xh)[Pro<T, FT, HT>::HK],
                                               const bf16x8 (&xl)[Pro<T, FT, HT>::HK],
                                               const bf16* w_hi, const bf16* w_lo, int lane) {
  using C = Pro<T, FT, HT>;
  const int h = lane >> 5;
  f32x16 acc = zero16();
#pragma unroll
  for (int kb = 0; kb < C::HK; ++kb) {
    const bf16x8 a = row_operand(w_hi, C::WP, 32 * ft + (lane & 31), 16 * kb, h);
    acc = mfma(a, xh[kb], acc);
    if constexpr (C::SPLIT) {
      acc = mfma(a, xl[kb], acc);
      acc = mfma(row_operand(w_lo, C::WP, 32 * ft + (lane & 31), 16 * kb, h), xh[kb], acc);
    }
  }
  return acc;
}

// Two softmax statistics (running max m, sum s of e^{x - m}) of one row merged.
__device__ __forceinline__ void merge_stats(float& m, float& s, float mo, float so) {
  const float m2 = fmaxf(m, mo);
  s = s * fexp(m - m2) + so * fexp(mo - m2);
  m = m2;
}

// Row statistics of the two softmaxes over the valid features (< f) in one
// pass over the feature tiles: per tile its maxima, the running sums rescaled
// to them (e^{x - m} as exp2 of one FMA), then the two lane halves' merged;
// returns the exp2 offsets of the two maps, -(m log2e + log2 sum): a feature's
// softmax value is then exp2(x log2e + offset) (for the negated map, of -x).
// PART: the last tile is partly padding (f < 32 FT), masked; without it there
// are no masks.
template <typename T, int FT, int HT, bool PART>
__device__ __forceinline__ void softmax_stats(const bf16x8 (&xh)[Pro<T, FT, HT>::HK],
                                              const bf16x8 (&xl)[Pro<T, FT, HT>::HK],
                                              const bf16* w_hi, const bf16* w_lo, int f,
                                              int lane, float& op, float& on) {
  const int h = lane >> 5;
  float mp = -1e30f, mn = -1e30f, sp = 0.f, sn = 0.f;
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const f32x16 acc = project_tile<T, FT, HT>(ft, xh, xl, w_hi, w_lo, lane);
    float tp = -1e30f, tn = -1e30f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool ok = !PART || 32 * ft + acc_row(r, h) < f;
      tp = fmaxf(tp, ok ? acc[r] : -1e30f);
      tn = fmaxf(tn, ok ? -acc[r] : -1e30f);
    }
    const float np = fmaxf(mp, tp), nn = fmaxf(mn, tn);
    const float cp = -np * LOG2E, cn = -nn * LOG2E;
    float ap = 0.f, an = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool ok = !PART || 32 * ft + acc_row(r, h) < f;
      ap += ok ? __builtin_amdgcn_exp2f(fmaf(acc[r], LOG2E, cp)) : 0.f;
      an += ok ? __builtin_amdgcn_exp2f(fmaf(acc[r], -LOG2E, cn)) : 0.f;
    }
    sp = sp * fexp(mp - np) + ap;
    sn = sn * fexp(mn - nn) + an;
    mp = np;
    mn = nn;
  }
  merge_stats(mp, sp, xhalf(mp), xhalf(sp));
  merge_stats(mn, sn, xhalf(mn), xhalf(sn));
  op = -(mp * LOG2E + __builtin_amdgcn_logf(sp));
  on = -(mn * LOG2E + __builtin_amdgcn_logf(sn));
}

struct RowPos {
  int b, l, head;
};

// row = (b L + l) heads + head (row counts stay below 2^31, checked by the host)
__device__ __forceinline__ RowPos decode(int row, int L, int heads) {
  const unsigned bl = (unsigned)row / (unsigned)heads;
  const unsigned b = bl / (unsigned)L;
  return RowPos{(int)b, (int)(bl - b * L), (int)(row - bl * heads)};
}


// Half `half` of the 2f-wide feature rows of a wave's 32 rows, staged in LDS
// ([32][pitch] bf16), to the rows' output rows in chunks of CH elements.
// Row r's output row (the obase of lane r, split in two ints) comes from
// lane r by a cross-lane read.
template <int CH>
__device__ __forceinline__ void copy_rows(const bf16* stage, int pitch, bf16* __restrict__ out,
                                          int ob_lo, int ob_hi, int row0, int nrows, int f,
                                          int half, int lane) {
  typedef __bf16 chunk_t __attribute__((ext_vector_type(CH)));
  const int cpr = f / CH;
  for (int i = lane; i < PRO_ROWS * cpr; i += 64) {
    const int r = i / cpr, c = CH * (i - r * cpr);
    const long base = ((long)__shfl(ob_hi, r) << 32) | (unsigned)__shfl(ob_lo, r);
    if (row0 + r >= nrows) continue;
    const chunk_t val = *reinterpret_cast<const chunk_t*>(stage + r * pitch + c);
    *reinterpret_cast<chunk_t*>(out + base * (2 * f) + half * f + c) = val;
  }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename T, int FT, int HT, bool PART>
__global__ __launch_bounds__(256, 2) void prologue_fwd_kernel(ProFwdArgs a) {
  using C = Pro<T, FT, HT>;
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* w_hi = reinterpret_cast<bf16*>(smem);
  bf16* w_lo = w_hi + C::W_ELEMS;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5;
  bf16* stage = w_hi + C::PARTS * C::W_ELEMS + wave * PRO_ROWS * C::SP;

  const bool kv = (int)blockIdx.x >= a.nq_wg;
  const int wg = kv ? blockIdx.x - a.nq_wg : blockIdx.x;
  const int nwg = kv ? gridDim.x - a.nq_wg : a.nq_wg;
  const int heads_in = kv ? a.Hkv : a.H;
  const int nrows = a.B * a.L * heads_in;
  const T* x = static_cast<const T*>(kv ? a.k : a.q);
  bf16* fout = kv ? a.fk : a.fq;
  bf16* rout = kv ? a.kr : a.qr;
  const T* cs = static_cast<const T*>(a.cos);
  const T* sn = static_cast<const T*>(a.sin);
  const int f = a.f, hd = C::HP, F2 = 2 * a.f;

  load_weight<T, FT, HT>(static_cast<const T*>(kv ? a.wk : a.wq), f, w_hi, w_lo);
  __syncthreads();

  for (int blk = wg; blk * PRO_BLOCK < nrows; blk += nwg) {
    const int row0 = blk * PRO_BLOCK + wave * PRO_ROWS;
    const int row = row0 + (lane & 31);
    const bool live = row < nrows;
    const RowPos pos = decode(live ? row : 0, a.L, heads_in);
    // its [B, heads_in, L, .] output row
    const long obase = ((long)pos.b * heads_in + pos.head) * a.L + pos.l;

    bf16x8 xh[C::HK], xl[C::HK];
    {
      // Every load of the row (x, the RoPE table rows, and for bf16 inputs v
      // of kv rows) is issued before anything is stored: as far as the
      // compiler knows the stores may alias the inputs, so a load written
      // after a store waits for it.  (fp32 rows load v after the RoPE stores:
      // its raw registers, twice the bf16 ones, would cost occupancy.)  A row
      // past the end reads row 0 (valid) and stores nothing; q rows read
      // their own x in place of v, unused.
      const long rrow = live ? row : 0;
      const long tab = ((long)pos.b * a.cos_bstride + pos.l) * hd + 8 * h;
      const T* xrow = x + rrow * hd + 8 * h;
      const T* vrow = (kv ? static_cast<const T*>(a.v) : x) + rrow * hd + 8 * h;
      Raw8<T> xr[C::HK], cr[C::HK], sr[C::HK], vr[C::HK];
#pragma unroll
      for (int kb = 0; kb < C::HK; ++kb) xr[kb] = load8r(xrow + 16 * kb);
#pragma unroll
      for (int kb = 0; kb < C::HK; ++kb) {
        cr[kb] = load8r(cs + tab + 16 * kb);
        sr[kb] = load8r(sn + tab + 16 * kb);
        if constexpr (sizeof(T) == 2) vr[kb] = load8r(vrow + 16 * kb);
      }
      float xf[C::HK][8];
#pragma unroll
      for (int kb = 0; kb < C::HK; ++kb) cvt8(xr[kb], xf[kb]);
      // RoPE (and the kv heads' v) from the fp32 row values: column
      // m = 16 kb + 8 h + e pairs with m + hd/2, the same column of kb + HK/2
      if (live) {
#pragma unroll
        for (int kb = 0; kb < C::HK / 2; ++kb) {
          const int kb2 = kb + C::HK / 2;
          float c1[8], s1[8], c2[8], s2[8];
          cvt8(cr[kb], c1);
          cvt8(sr[kb], s1);
          cvt8(cr[kb2], c2);
          cvt8(sr[kb2], s2);
          bf16x8 o1, o2;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            o1[e] = to_bf16(xf[kb][e] * c1[e] - xf[kb2][e] * s1[e]);
            o2[e] = to_bf16(xf[kb2][e] * c2[e] + xf[kb][e] * s2[e]);
          }
          bf16* dst = rout + obase * hd;
          *reinterpret_cast<bf16x8*>(dst + 16 * kb + 8 * h) = o1;
          *reinterpret_cast<bf16x8*>(dst + 16 * kb2 + 8 * h) = o2;
        }
        if (kv) {
          if constexpr (sizeof(T) != 2) {
#pragma unroll
            for (int kb = 0; kb < C::HK; ++kb) vr[kb] = load8r(vrow + 16 * kb);
          }
#pragma unroll
          for (int kb = 0; kb < C::HK; ++kb) {
            float vf[8];
            cvt8(vr[kb], vf);
            *reinterpret_cast<bf16x8*>(a.vo + obase * hd + 16 * kb + 8 * h) = to_bf8(vf);
          }
        }
      }
#pragma unroll
      for (int kb = 0; kb < C::HK; ++kb) {
        xh[kb] = to_bf8(xf[kb]);
        if constexpr (C::SPLIT) xl[kb] = low8(xf[kb], xh[kb]);
      }
    }
    // fq == nullptr: q rows stop at RoPE (the GLA walk forms their feature
    // map itself, lz_gla_fwd_phi); fout is uniform per workgroup
    if (fout == nullptr) continue;
    float cp, cn;
    softmax_stats<T, FT, HT, PART>(xh, xl, w_hi, w_lo, f, lane, cp, cn);

    // the two halves of the feature row, staged through LDS for row-contiguous stores
    const int ob_lo = (int)(obase & 0xffffffff), ob_hi = (int)(obase >> 32);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
#pragma unroll
      for (int ft = 0; ft < FT; ++ft) {
        const f32x16 acc = project_tile<T, FT, HT>(ft, xh, xl, w_hi, w_lo, lane);
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          bf16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float s = acc[4 * q4 + e];
            o[e] = to_bf16(half == 0 ? __builtin_amdgcn_exp2f(fmaf(s, LOG2E, cp))
                                     : __builtin_amdgcn_exp2f(fmaf(s, -LOG2E, cn)));
          }
          *reinterpret_cast<bf16x4*>(stage + (lane & 31) * C::SP + 32 * ft + 8 * q4 + 4 * h) = o;
        }
      }
      wave_sync();
      if (f % 8 == 0)
        copy_rows<8>(stage, C::SP, fout, ob_lo, ob_hi, row0, nrows, f, half, lane);
      else
        copy_rows<4>(stage, C::SP, fout, ob_lo, ob_hi, row0, nrows, f, half, lane);
      wave_sync();
    }
  }
}

// ---------------------------------------------------------------------------
// backward
//
// A workgroup takes blocks of 128 rows.  Its 4 NWF waves are (row group rg,
// feature group fh): wave (rg, fh) owns rows 32 rg .. 32 rg + 31 (one per lane
// column of its MFMA tiles) and feature tiles fh, fh + NWF, ... (FTW = FT / NWF
// of them) of both maps.  Splitting a row's features over NWF = 2 waves
// halves what a lane keeps in registers through the Jacobian, which is what
// lets two waves share a SIMD at f = 128.  Per block:
//   1. x rows -> LDS (bf16 hi, and lo for fp32 inputs), coalesced; each lane
//      reads its row's MFMA operands back;
//   2. softmax statistics of both feature maps over the wave's tiles in one
//      pass (per-tile maxima, running rescaled sums), combined across the
//      feature groups through LDS;
//   3. per local tile s: the gradient rows' 32 dp and 32 dn values of tile s of
//      every feature group, summed over the group's heads in fp32, are
//      gathered by the whole workgroup with 16-byte loads into an fp32 LDS
//      stage (the next tile's loads in flight meanwhile), and each lane forms
//      A = p dp - n dn and its shares of <p, dp>, <n, dn> (summed across the
//      feature groups through LDS afterwards);
//   4. dxw = A + n <n,dn> - p <p,dp> per tile: the wave's share of
//      dx_phi^T = W^T dxw^T (MFMA, hi and lo parts of dxw), dxw hi -> the dW
//      tile in LDS;
//   5. dW += dxw^T x over the block (hi, then lo), through LDS transpose reads;
//   6. the dx_phi shares -> LDS, and dx = their sum + rope^T(drope) (plus the
//      summed dv for the kv rows) in a coalesced row layout, 8 columns per item.
// The stage, the dW tile and the dx tile share one LDS buffer.
// ---------------------------------------------------------------------------
constexpr int imax(int a, int b) { return a > b ? a : b; }

template <typename T, int FT, int HT>
struct ProBwd {
  using C = Pro<T, FT, HT>;
  static constexpr int FP = C::FP, HP = C::HP, HK = C::HK, WP = C::WP, PARTS = C::PARTS;
  // feature groups: two where a row has two or more feature tiles and the
  // per-group dx shares fit the LDS (head_dim <= 64)
  static constexpr int NWF = FT >= 2 && HT <= 2 ? 2 : 1;
  static constexpr int FTW = FT / NWF;                   // feature tiles per wave
  static constexpr int NW = PRO_WAVES * NWF, NT = 64 * NW;
  static constexpr int QP = lds_pitch(HP);    // x tiles [128][QP] bf16
  static constexpr int DP = lds_pitch(FP);    // dW tile [128][DP] bf16
  static constexpr int SP = 64 * NWF + 4;     // stage [128][SP] fp32: per group 32 dp, 32 dn
  static constexpr int AP = HP + 4;           // dx shares [NWF][128][AP] fp32
  static constexpr int BUF = imax(PRO_BLOCK * SP * 4, PRO_BLOCK * DP * 2);
  static constexpr int OFF_X = PARTS * FP * WP * 2;
  static constexpr int OFF_B = OFF_X + PARTS * PRO_BLOCK * QP * 2;
  // the dx shares take the buffer when they fit there, else they also span
  // the x tiles (then the next block waits for the epilogue before writing x)
  static constexpr int DX = NWF * PRO_BLOCK * AP * 4;
  static constexpr bool DX_OVER_X = DX > BUF;
  static constexpr int OFF_DX = DX_OVER_X ? OFF_X : OFF_B;
  static constexpr int OFF_RED = imax(OFF_B + BUF, OFF_DX + DX);   // [NWF][4][128] row stats
  static constexpr int LDS = OFF_RED + NWF * 4 * PRO_BLOCK * 4;
  static constexpr int OCC = LDS <= 80 * 1024 && NW == 4 ? 2 : 1;   // workgroups per CU
  static constexpr int IPR = 8 * NWF;                    // stage items per row
  static constexpr int GI = PRO_BLOCK * IPR / NT;        // stage items per thread
  static constexpr int RSTEP = NT / IPR;                 // rows between a thread's items
  static constexpr int XI = PRO_BLOCK * (HP / 8) / NT;   // x / dx items per thread
  static_assert(GI * RSTEP * IPR == PRO_BLOCK * IPR && RSTEP == 32, "item mapping");
  static_assert(XI * NT == PRO_BLOCK * (HP / 8), "row items");
  static constexpr bool FITS = LDS <= 160 * 1024;   // instantiated for launch only when it fits
  // the next block's x rows and the epilogue's first-head operands are issued
  // a phase early (their latency then hides behind the dW passes): where one
  // workgroup per CU leaves the registers for them (bf16, head_dim <= 64);
  // elsewhere the held loads push the kernel into spills
  static constexpr bool PRE = OCC == 1 && HT <= 2 && !C::SPLIT;
  // heads whose gradient loads are issued a tile ahead: four where one wave
  // per SIMD has the registers for them, one in the split form with PRE (the
  // q blocks' only head: 1 % at config 5), none elsewhere (the two-workgroup
  // forms' second wave per SIMD hides the load latency instead, and held
  // loads push them into spills; nor at FT = HT = 4, where a wave's own tiles
  // already take every register)
  static constexpr int GQ = OCC == 1 && NWF == 1 && FT * HT < 16 ? 4 : (PRE ? 1 : 0);
  static constexpr int GQR = GQ > 0 ? GQ : 1;            // raw register sets held
};

template <typename T>
__device__ __forceinline__ void store8v(T* __restrict__ p, const float (&x)[8]) {
  if constexpr (sizeof(T) == 2) {
    bf16x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = to_bf16(x[e]);
    *reinterpret_cast<bf16x8*>(p) = o;
  } else {
    *reinterpret_cast<f32x4*>(p) = f32x4{x[0], x[1], x[2], x[3]};
    *reinterpret_cast<f32x4*>(p + 4) = f32x4{x[4], x[5], x[6], x[7]};
  }
}

// PART: f < 32 FT, so the last feature tile is partly padding and its
// features past f are masked out (the instantiation without it carries no
// masks at all).
template <typename T, int FT, int HT, bool PART>
__global__ __launch_bounds__((ProBwd<T, FT, HT>::NT), (ProBwd<T, FT, HT>::OCC)) void
prologue_bwd_kernel(ProBwdArgs a) {
  using K = ProBwd<T, FT, HT>;
  constexpr int FP = K::FP, HP = K::HP, HK = K::HK, SP = K::SP, AP = K::AP;
  constexpr int NWF = K::NWF, FTW = K::FTW, NW = K::NW, NT = K::NT;
  constexpr bool SPLIT = Pro<T, FT, HT>::SPLIT;
  constexpr int TILES = FT * HT;
  constexpr int OWN = (TILES + NW - 1) / NW;   // dW tiles per wave
  constexpr int H8 = HP / 8;                   // 8-column items per hd row
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* w_hi = reinterpret_cast<bf16*>(smem);
  bf16* w_lo = w_hi + FP * K::WP;
  bf16* x_hi = reinterpret_cast<bf16*>(smem + K::OFF_X);
  bf16* x_lo = x_hi + PRO_BLOCK * K::QP;
  float* stage = reinterpret_cast<float*>(smem + K::OFF_B);
  bf16* d_l = reinterpret_cast<bf16*>(smem + K::OFF_B);
  float* dx_l = reinterpret_cast<float*>(smem + K::OFF_DX);
  float* red = reinterpret_cast<float*>(smem + K::OFF_RED);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, h = lane >> 5;
  const int rg = wave % PRO_WAVES, fh = wave / PRO_WAVES;   // row group, feature group
  const int lrow = rg * PRO_ROWS + (lane & 31);             // this lane's row in the tiles
  // local tile s of feature group g is feature tile s NWF + g: the groups'
  // tiles interleave, so one pass over local tile s gathers the adjacent
  // 32-feature tiles 2s and 2s + 1 of a gradient row, a whole 128-byte line of
  // it (blocked tiles read half lines per pass, and the other halves came back
  // from HBM a pass later, evicted meanwhile)
  auto ftile = [](int g, int s) { return s * NWF + g; };

  const T* cs = static_cast<const T*>(a.cos);
  const T* sn = static_cast<const T*>(a.sin);
  const int f = a.f, hd = HP, half_hd = HP / 2, F2 = 2 * a.f;
  // gradient items are whole 16-byte pieces (always without a partial tile:
  // then f is a multiple of 32)
  const bool vec = !PART || (f & 7) == 0;

  // stage items of this thread: rows tid / IPR + 32 i of a block; item k of a
  // row covers features 8 (k & 3) .. +8 of tile ftile(k / 8, s) of the dp
  // ((k / 4) & 1 == 0) or dn map, at stage column 8 k
  const int k = tid % K::IPR, sgrp = k >> 3, shalf = (k >> 2) & 1, scol = 8 * (k & 3);
  const int srow = tid / K::IPR;

  // this workgroup's partial dW [FP][HP] of role r: lane = column, registers = rows
  auto flush = [&](const f32x16 (&acc)[OWN], int r, bool zero) {
    float* part = a.part + ((size_t)r * gridDim.x + blockIdx.x) * FP * HP;
#pragma unroll
    for (int i = 0; i < OWN; ++i) {
      const int t = wave + NW * i;
      if (t < TILES) {
        const int ft = t / HT, ht = t % HT;
#pragma unroll
        for (int r2 = 0; r2 < 16; ++r2)
          part[(32 * ft + acc_row(r2, h)) * HP + 32 * ht + (lane & 31)] = zero ? 0.f : acc[i][r2];
      }
    }
  };

  // One grid over the q blocks, then the kv blocks: workgroup w takes blocks
  // w, w + G, ... of that list, so it switches role at most once and every
  // workgroup gets its share of both (kv blocks carry the group's gradients).
  // Workgroups of odd index take theirs in reverse order, kv blocks first: at
  // any time about half the CUs then walk kv blocks (four heads' gradients
  // each, bandwidth-heavy) while the others walk q blocks (round-trip bound),
  // where in list order all walked the q blocks and then all the kv blocks.
  bool kv = false;
  int role = -1, heads_in = 0, group = 1, nrows = 0;
  const bf16 *dphi = nullptr, *drope = nullptr;
  T* dx = nullptr;
  f32x16 dw[OWN];
#pragma unroll
  for (int i = 0; i < OWN; ++i) dw[i] = zero16();

  const int nb = a.nbq + a.nbk;
  // x rows of block jb (this thread's XI items): with PRE issued during the
  // previous block's dW passes, so the next block starts with its rows in
  // registers; else at the block's start.  Rows past the end read the last
  // row's address and are zeroed at use.
  auto x_items = [&](int jb, Raw8<T> (&dst)[K::XI]) {
    const bool kvb = jb >= a.nbq;
    const T* xs = static_cast<const T*>(kvb ? a.k : a.q);
    const int nr = a.B * a.L * (kvb ? a.Hkv : a.H);
    const int r0 = (kvb ? jb - a.nbq : jb) * PRO_BLOCK;
#pragma unroll
    for (int i = 0; i < K::XI; ++i) {
      const int idx = tid + NT * i, r = idx / H8, m0 = 8 * (idx % H8);
      dst[i] = load8r(xs + (long)min(r0 + r, nr - 1) * hd + m0);
    }
  };
  const int G = gridDim.x, w = blockIdx.x;
  const int nmine = w < nb ? (nb - w + G - 1) / G : 0;   // this workgroup's blocks
  const bool rev = (w & 1) != 0;
  auto block_of = [&](int kk) { return w + (rev ? nmine - 1 - kk : kk) * G; };
  bool taken[2] = {false, false};   // roles whose partial has been written
  Raw8<T> xpre[K::XI];
  if (K::PRE && nmine > 0) x_items(block_of(0), xpre);
  for (int kk = 0; kk < nmine; ++kk) {
    const int j = block_of(kk);
    if constexpr (!K::PRE) x_items(j, xpre);
    const int r_j = j < a.nbq ? 0 : 1;
    if (r_j != role) {   // uniform; the W tile's readers passed the last block's barriers
      if (role >= 0) {   // the role in hand is done: its partial
        flush(dw, role, false);
        taken[role] = true;
#pragma unroll
        for (int i = 0; i < OWN; ++i) dw[i] = zero16();
      }
      role = r_j;
      kv = role == 1;
      heads_in = kv ? a.Hkv : a.H;
      group = kv ? a.H / a.Hkv : 1;
      nrows = a.B * a.L * heads_in;
      dphi = kv ? a.dfk : a.dfq;
      drope = kv ? a.dkr : a.dqr;
      dx = static_cast<T*>(kv ? a.dk : a.dq);
      load_weight<T, FT, HT>(static_cast<const T*>(kv ? a.wk : a.wq), f, w_hi, w_lo);
    }
    const int row0 = (kv ? j - a.nbq : j) * PRO_BLOCK;

    // rows of this thread's stage items: [B, H, L, 2f] element offset of
    // their first head's gradient row (-1: row past the end)
    long gbase[K::GI];
#pragma unroll
    for (int i = 0; i < K::GI; ++i) {
      const int row = row0 + srow + 32 * i;
      if (row < nrows) {
        const RowPos pos = decode(row, a.L, heads_in);
        gbase[i] = (((long)pos.b * a.H + pos.head * group) * a.L + pos.l) * F2 + shalf * f;
      } else {
        gbase[i] = -1;
      }
    }
    // Gradient items of local tile s: the loads of the first GQ heads are
    // issued a tile ahead (raw, 16 bytes each) and summed when the tile is
    // staged; heads past GQ are loaded and added then.  The 16-byte loads are
    // nontemporal: nothing reads these gradient rows again (config 5:
    // 325.3 -> 320.7 us; the same policy on the x-row and epilogue loads
    // gained nothing more, and the loads written through a helper function
    // came out with 16 spilled registers instead of 6).
    auto item_ok = [&](int i, int c) { return gbase[i] >= 0 && (!PART || c < f); };
    auto issue = [&](int s, uint4 (&raw)[K::GQR][K::GI]) {
      const int c = 32 * ftile(sgrp, s) + scol;
#pragma unroll
      for (int g = 0; g < K::GQ; ++g)
#pragma unroll
        for (int i = 0; i < K::GI; ++i)
          if (g < group) {   // uniform
            const bf16* p = dphi + (gbase[i] + (long)g * a.L * F2 + c);
            if (vec) {
              raw[g][i] = __builtin_bit_cast(uint4, __builtin_nontemporal_load(
                                                       reinterpret_cast<const u32x4*>(item_ok(i, c) ? p : dphi)));
            } else {
              const uint2 lo = *reinterpret_cast<const uint2*>(item_ok(i, c) ? p : dphi);
              const uint2 hi = *reinterpret_cast<const uint2*>(item_ok(i, c + 4) ? p + 4 : dphi);
              raw[g][i] = uint4{lo.x, lo.y, hi.x, hi.y};
            }
          }
    };
    // Heads past GQ: per head, the loads of all GI items are issued before any
    // is summed (each item's heads are still summed in head order), so GI
    // loads per thread are in flight instead of one.
    auto gather = [&](int s, const uint4 (&raw)[K::GQR][K::GI], float (&g8)[K::GI][8]) {
      const int c = 32 * ftile(sgrp, s) + scol;
      bool ok0[K::GI], ok1[K::GI];
#pragma unroll
      for (int i = 0; i < K::GI; ++i) {
#pragma unroll
        for (int e = 0; e < 8; ++e) g8[i][e] = 0.f;
        ok0[i] = item_ok(i, c);
        ok1[i] = item_ok(i, c + 4);
#pragma unroll
        for (int g = 0; g < K::GQ; ++g)
          if (g < group) {
            const bf16x8 v = __builtin_bit_cast(bf16x8, raw[g][i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) g8[i][e] += (e < 4 ? ok0[i] : ok1[i]) ? to_f32(v[e]) : 0.f;
          }
      }
      for (int g = K::GQ; g < group; ++g) {
        uint4 v[K::GI];
#pragma unroll
        for (int i = 0; i < K::GI; ++i) {
          const bf16* p = dphi + (gbase[i] + (long)g * a.L * F2 + c);
          if (vec) {
            v[i] = __builtin_bit_cast(
                uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ok0[i] ? p : dphi)));
          } else {
            const uint2 lo = *reinterpret_cast<const uint2*>(ok0[i] ? p : dphi);
            const uint2 hi = *reinterpret_cast<const uint2*>(ok1[i] ? p + 4 : dphi);
            v[i] = uint4{lo.x, lo.y, hi.x, hi.y};
          }
        }
#pragma unroll
        for (int i = 0; i < K::GI; ++i) {
          const bf16x8 x8 = __builtin_bit_cast(bf16x8, v[i]);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            g8[i][e] += (e < 4 ? ok0[i] : ok1[i]) ? to_f32(x8[e]) : 0.f;
        }
      }
    };
    uint4 raw[K::GQR][K::GI];
    if constexpr (K::GQ > 0) issue(0, raw);

    // ---- 1. x rows -> LDS; this lane's operands ------------------------------
#pragma unroll
    for (int i = 0; i < K::XI; ++i) {
      const int idx = tid + NT * i, r = idx / H8, m0 = 8 * (idx % H8);
      float xf[8];
      cvt8(xpre[i], xf);
      if (row0 + r >= nrows) {
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = 0.f;
      }
      const bf16x8 hi = to_bf8(xf);
      *reinterpret_cast<bf16x8*>(x_hi + r * K::QP + m0) = hi;
      if constexpr (SPLIT) *reinterpret_cast<bf16x8*>(x_lo + r * K::QP + m0) = low8(xf, hi);
    }
    __syncthreads();   // x tiles (and, after a role switch, W); the last block's epilogue is done
    bf16x8 xh[HK], xl[HK];
#pragma unroll
    for (int kb = 0; kb < HK; ++kb) {
      xh[kb] = row_operand(x_hi, K::QP, lrow, 16 * kb, h);
      if constexpr (SPLIT) xl[kb] = row_operand(x_lo, K::QP, lrow, 16 * kb, h);
    }

    // ---- 2. softmax statistics: maxima and sums in one pass -----------------
    float mp = -1e30f, mn = -1e30f, sp = 0.f, sn_ = 0.f;
#pragma unroll
    for (int s = 0; s < FTW; ++s) {
      const int ft = ftile(fh, s);
      const f32x16 acc = project_tile<T, FT, HT>(ft, xh, xl, w_hi, w_lo, lane);
      // features past f (padding of the last tile) drop out through
      // selects, not branches: their exponentials are of -inf
      float tp = -1e30f, tn = -1e30f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool ok = !PART || 32 * ft + acc_row(r, h) < f;
        tp = fmaxf(tp, ok ? acc[r] : -1e30f);
        tn = fmaxf(tn, ok ? -acc[r] : -1e30f);
      }
      const float np = fmaxf(mp, tp), nn = fmaxf(mn, tn);
      const float cp = -np * LOG2E, cn = -nn * LOG2E;   // e^{x - m} = exp2(x log2e - m log2e)
      float ap = 0.f, an = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool ok = !PART || 32 * ft + acc_row(r, h) < f;
        ap += ok ? __builtin_amdgcn_exp2f(fmaf(acc[r], LOG2E, cp)) : 0.f;
        an += ok ? __builtin_amdgcn_exp2f(fmaf(acc[r], -LOG2E, cn)) : 0.f;
      }
      sp = sp * fexp(mp - np) + ap;
      sn_ = sn_ * fexp(mn - nn) + an;
      mp = np;
      mn = nn;
    }
    // the other lane half holds other features of the row ...
    merge_stats(mp, sp, xhalf(mp), xhalf(sp));
    merge_stats(mn, sn_, xhalf(mn), xhalf(sn_));
    if constexpr (NWF > 1) {   // ... and the other feature group the rest
      float* mine = red + fh * 4 * PRO_BLOCK;
      if (h == 0) {
        mine[lrow] = mp;
        mine[PRO_BLOCK + lrow] = sp;
        mine[2 * PRO_BLOCK + lrow] = mn;
        mine[3 * PRO_BLOCK + lrow] = sn_;
      }
      __syncthreads();
      const float* other = red + (1 - fh) * 4 * PRO_BLOCK;
      const float omp = other[lrow], osp = other[PRO_BLOCK + lrow];
      const float omn = other[2 * PRO_BLOCK + lrow], osn = other[3 * PRO_BLOCK + lrow];
      // both groups merge in the same order (group 0 first): identical results
      if (fh == 0) {
        merge_stats(mp, sp, omp, osp);
        merge_stats(mn, sn_, omn, osn);
      } else {
        float m0 = omp, s0 = osp, n0 = omn, t0 = osn;
        merge_stats(m0, s0, mp, sp);
        merge_stats(n0, t0, mn, sn_);
        mp = m0, sp = s0, mn = n0, sn_ = t0;
      }
    }
    // p = e^{x - mp} / sp = exp2(x log2e - (mp log2e + log2 sp)), n likewise:
    // one FMA and the hardware exp2 per feature
    const float lp = -(mp * LOG2E + __builtin_amdgcn_logf(sp));
    const float ln_ = -(mn * LOG2E + __builtin_amdgcn_logf(sn_));

    // ---- 3. A = p dp - n dn per feature tile, <p, dp>, <n, dn> ---------------
    f32x16 A[FTW];
    float s_p = 0.f, s_n = 0.f;
#pragma unroll
    for (int s = 0; s < FTW; ++s) {
      float g8[K::GI][8];
      gather(s, raw, g8);
      if (K::GQ > 0 && s + 1 < FTW) issue(s + 1, raw);   // in flight while this tile computes
      __syncthreads();   // the previous tile's readers of the buffer (and red) are done
#pragma unroll
      for (int i = 0; i < K::GI; ++i) {
        float* dst = stage + (srow + 32 * i) * SP + 8 * k;
        *reinterpret_cast<f32x4*>(dst) = f32x4{g8[i][0], g8[i][1], g8[i][2], g8[i][3]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{g8[i][4], g8[i][5], g8[i][6], g8[i][7]};
      }
      __syncthreads();
      const f32x16 acc = project_tile<T, FT, HT>(ftile(fh, s), xh, xl, w_hi, w_lo, lane);
      const float* srow_l = stage + lrow * SP + 64 * fh;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const f32x4 dp = *reinterpret_cast<const f32x4*>(srow_l + 8 * q4 + 4 * h);
        const f32x4 dn = *reinterpret_cast<const f32x4*>(srow_l + 32 + 8 * q4 + 4 * h);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * q4 + e;
          const float pd = __builtin_amdgcn_exp2f(fmaf(acc[r], LOG2E, lp)) * dp[e];
          const float nd = __builtin_amdgcn_exp2f(fmaf(acc[r], -LOG2E, ln_)) * dn[e];
          A[s][r] = pd - nd;
          s_p += pd;
          s_n += nd;
        }
      }
    }
    s_p += xhalf(s_p);
    s_n += xhalf(s_n);
    if constexpr (NWF > 1) {
      if (h == 0) {
        red[fh * 4 * PRO_BLOCK + lrow] = s_p;
        red[fh * 4 * PRO_BLOCK + PRO_BLOCK + lrow] = s_n;
      }
    }
    __syncthreads();   // every lane is done with the stage (and the shares are in red)
    if constexpr (NWF > 1) {   // group 0's share first, in both groups
      const float p0 = red[lrow], p1 = red[4 * PRO_BLOCK + lrow];
      const float n0 = red[PRO_BLOCK + lrow], n1 = red[5 * PRO_BLOCK + lrow];
      s_p = p0 + p1;
      s_n = n0 + n1;
    }

    // ---- 4. dxw; the wave's share of dx_phi^T = W^T dxw^T; dxw hi -> dW tile --
    f32x16 dacc[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) dacc[ht] = zero16();
    bf16x4 dlo[FTW][4];
#pragma unroll
    for (int s = 0; s < FTW; ++s) {
      const int ft = ftile(fh, s);
      const f32x16 acc = project_tile<T, FT, HT>(ft, xh, xl, w_hi, w_lo, lane);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(acc[r], LOG2E, lp));
        const float n = __builtin_amdgcn_exp2f(fmaf(acc[r], -LOG2E, ln_));
        A[s][r] = !PART || 32 * ft + acc_row(r, h) < f ? A[s][r] + n * s_n - p * s_p : 0.f;
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 dh = acc_operand(A[s], kb), dl = acc_operand_lo(A[s], kb);
#pragma unroll
        for (int ht = 0; ht < HT; ++ht) {
          const bf16x8 w = tr_operand(w_hi, K::WP, 32 * ft + 16 * kb, 32 * ht, lane);
          dacc[ht] = mfma(w, dh, dacc[ht]);
          dacc[ht] = mfma(w, dl, dacc[ht]);
          if constexpr (SPLIT)
            dacc[ht] = mfma(tr_operand(w_lo, K::WP, 32 * ft + 16 * kb, 32 * ht, lane), dh,
                            dacc[ht]);
        }
      }
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        bf16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v = A[s][4 * q4 + e];
          o[e] = to_bf16(v);
          dlo[s][q4][e] = to_bf16(v - to_f32(o[e]));
        }
        *reinterpret_cast<bf16x4*>(d_l + lrow * K::DP + 32 * ft + 8 * q4 + 4 * h) = o;
      }
    }

    // ---- with PRE: the epilogue operands of the group's first head and the
    // RoPE tables, issued before the dW passes, whose barriers and MFMA work
    // then cover their latency (the later heads of a kv group load in phase
    // 6), and the next block's x rows.  Rows past the end read the last row's
    // addresses and are not stored.
    // dx[m] = dr[m] cos[m] + dr[m + hd/2] sin[m + hd/2] for m < hd/2,
    //         dr[m] cos[m] - dr[m - hd/2] sin[m - hd/2] otherwise (drope summed
    // over the group's heads); the kv rows also sum dv (and dv2) over the group.
    // The dv loads of a q row (and dv2's when there is none) read a valid
    // address whose value is dropped, so there is no branch between them.
    const bool use_dv = kv, use_dv2 = kv && a.dv2 != nullptr;
    constexpr int EXI = K::PRE ? K::XI : 1;
    long ebase[EXI];
    Raw8<T> ec[EXI], es[EXI];
    bf16x8 er0[EXI], er1[EXI], ev0[EXI], ev1[EXI];
#pragma unroll
    for (int i = 0; i < (K::PRE ? K::XI : 0); ++i) {
      const int idx = tid + NT * i, r = idx / H8, m0 = 8 * (idx % H8);
      const int row = min(row0 + r, nrows - 1);
      const RowPos pos = decode(row, a.L, heads_in);
      ebase[i] = ((long)pos.b * a.H + pos.head * group) * a.L + pos.l;
      const int mp2 = m0 < half_hd ? m0 + half_hd : m0 - half_hd;
      const long tab = ((long)pos.b * a.cos_bstride + pos.l) * hd;
      const long o = ebase[i] * hd;
      er0[i] = *reinterpret_cast<const bf16x8*>(drope + o + m0);
      er1[i] = *reinterpret_cast<const bf16x8*>(drope + o + mp2);
      ev0[i] = *reinterpret_cast<const bf16x8*>(use_dv ? a.dv + o + m0 : drope + o + m0);
      ev1[i] = *reinterpret_cast<const bf16x8*>(use_dv2 ? a.dv2 + o + m0 : drope + o + m0);
      ec[i] = load8r(cs + tab + m0);
      es[i] = load8r(sn + tab + mp2);
    }
    if (K::PRE && kk + 1 < nmine) x_items(block_of(kk + 1), xpre);

    // ---- 5. dW += dxw^T x over the block: dxw hi, then lo --------------------
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      if (part == 1) {
#pragma unroll
        for (int s = 0; s < FTW; ++s)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            *reinterpret_cast<bf16x4*>(d_l + lrow * K::DP + 32 * ftile(fh, s) + 8 * q4 + 4 * h) =
                dlo[s][q4];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < OWN; ++i) {
        const int t = wave + NW * i;
        if (t < TILES) {
          const int ft = t / HT, ht = t % HT;
#pragma unroll 2
          for (int ks = 0; ks < PRO_BLOCK / 16; ++ks) {
            const bf16x8 d = tr_operand(d_l, K::DP, 16 * ks, 32 * ft, lane);
            dw[i] = mfma(d, tr_operand(x_hi, K::QP, 16 * ks, 32 * ht, lane), dw[i]);
            if (SPLIT && part == 0)
              dw[i] = mfma(d, tr_operand(x_lo, K::QP, 16 * ks, 32 * ht, lane), dw[i]);
          }
        }
      }
      __syncthreads();
    }

    // ---- 6. dx = sum of the dx_phi shares + rope^T(drope) (+ dv sums) --------
    {
      float* mine = dx_l + fh * PRO_BLOCK * AP;
#pragma unroll
      for (int ht = 0; ht < HT; ++ht)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          *reinterpret_cast<f32x4*>(mine + lrow * AP + 32 * ht + 8 * q4 + 4 * h) =
              f32x4{dacc[ht][4 * q4], dacc[ht][4 * q4 + 1], dacc[ht][4 * q4 + 2],
                    dacc[ht][4 * q4 + 3]};
    }
    __syncthreads();
    if constexpr (K::PRE) {
#pragma unroll
      for (int i = 0; i < K::XI; ++i) {
        const int idx = tid + NT * i, r = idx / H8, m0 = 8 * (idx % H8);
        const int row = row0 + r;
        const int mp2 = m0 < half_hd ? m0 + half_hd : m0 - half_hd;
        const float sign = m0 < half_hd ? 1.f : -1.f;
        float dr[8], dr2[8], dvs[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dr[e] = to_f32(er0[i][e]);
          dr2[e] = to_f32(er1[i][e]);
          dvs[e] = use_dv ? to_f32(ev0[i][e]) : 0.f;
          dvs[e] += use_dv2 ? to_f32(ev1[i][e]) : 0.f;
        }
        // the group's later heads: a head's four loads issue before any of them is summed
#pragma unroll 2
        for (int g = 1; g < group; ++g) {
          const long o = (ebase[i] + (long)g * a.L) * hd;
          const bf16x8 r0 = *reinterpret_cast<const bf16x8*>(drope + o + m0);
          const bf16x8 r1 = *reinterpret_cast<const bf16x8*>(drope + o + mp2);
          const bf16x8 v0 = *reinterpret_cast<const bf16x8*>(use_dv ? a.dv + o + m0 : drope + o + m0);
          const bf16x8 v1 = *reinterpret_cast<const bf16x8*>(use_dv2 ? a.dv2 + o + m0 : drope + o + m0);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            dr[e] += to_f32(r0[e]);
            dr2[e] += to_f32(r1[e]);
            dvs[e] += use_dv ? to_f32(v0[e]) : 0.f;
            dvs[e] += use_dv2 ? to_f32(v1[e]) : 0.f;
          }
        }
        float c[8], s2[8], out[8];
        cvt8(ec[i], c);
        cvt8(es[i], s2);
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = dr[e] * c[e] + sign * dr2[e] * s2[e];
#pragma unroll
        for (int g2 = 0; g2 < NWF; ++g2) {   // the shares in group order
          const float* dxr = dx_l + (g2 * PRO_BLOCK + r) * AP + m0;
#pragma unroll
          for (int e = 0; e < 8; ++e) out[e] += dxr[e];
        }
        if (row < nrows) {
          store8v(dx + (long)row * hd + m0, out);
          if (kv) store8v(static_cast<T*>(a.dvo) + (long)row * hd + m0, dvs);
        }
      }
    } else {
      // Two items' loads overlap (unrolled by 2): the Jacobian's registers are free here.
#pragma unroll 2
      for (int i = 0; i < K::XI; ++i) {
        const int idx = tid + NT * i, r = idx / H8, m0 = 8 * (idx % H8);
        const int row = row0 + r;
        if (row >= nrows) continue;
        const RowPos pos = decode(row, a.L, heads_in);
        const long obase = ((long)pos.b * a.H + pos.head * group) * a.L + pos.l;
        const int mp2 = m0 < half_hd ? m0 + half_hd : m0 - half_hd;
        const float sign = m0 < half_hd ? 1.f : -1.f;
        float dr[8], dr2[8], dvs[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) dr[e] = dr2[e] = dvs[e] = 0.f;
        // a head's four loads issue before any of them is summed; the dv loads
        // of a q row (and dv2's when there is none) read a valid address whose
        // value is dropped, so there is no branch between them
#pragma unroll 2
        for (int g = 0; g < group; ++g) {
          const long o = (obase + (long)g * a.L) * hd;
          const bf16x8 r0 = *reinterpret_cast<const bf16x8*>(drope + o + m0);
          const bf16x8 r1 = *reinterpret_cast<const bf16x8*>(drope + o + mp2);
          const bf16x8 v0 = *reinterpret_cast<const bf16x8*>(use_dv ? a.dv + o + m0 : drope + o + m0);
          const bf16x8 v1 = *reinterpret_cast<const bf16x8*>(use_dv2 ? a.dv2 + o + m0 : drope + o + m0);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            dr[e] += to_f32(r0[e]);
            dr2[e] += to_f32(r1[e]);
            dvs[e] += use_dv ? to_f32(v0[e]) : 0.f;
            dvs[e] += use_dv2 ? to_f32(v1[e]) : 0.f;
          }
        }
        const long tab = ((long)pos.b * a.cos_bstride + pos.l) * hd;
        float c[8], s2[8], out[8];
        load8f(cs + tab + m0, c);
        load8f(sn + tab + mp2, s2);
#pragma unroll
        for (int e = 0; e < 8; ++e) out[e] = dr[e] * c[e] + sign * dr2[e] * s2[e];
#pragma unroll
        for (int g2 = 0; g2 < NWF; ++g2) {   // the shares in group order
          const float* dxr = dx_l + (g2 * PRO_BLOCK + r) * AP + m0;
#pragma unroll
          for (int e = 0; e < 8; ++e) out[e] += dxr[e];
        }
        store8v(dx + (long)row * hd + m0, out);
        if (kv) store8v(static_cast<T*>(a.dvo) + (long)row * hd + m0, dvs);
      }
    }
    if constexpr (K::DX_OVER_X) __syncthreads();
  }
  // the role in hand (its partial), and zeros for a role never taken
  if (role >= 0) {
    flush(dw, role, false);
    taken[role] = true;
  }
  if (!taken[0]) flush(dw, 0, true);
  if (!taken[1]) flush(dw, 1, true);
}

// dW[i][c] = sum over a role's workgroups of their partials.  A block takes 64
// consecutive (i, c) entries; its 4 waves sum interleaved quarters of the
// workgroups (8 independent loads in flight per lane), then wave 0 adds the
// four quarter sums in a fixed order: deterministic.
__global__ __launch_bounds__(256) void prologue_dw_reduce_kernel(const float* __restrict__ part,
                                                                 float* __restrict__ dwq,
                                                                 float* __restrict__ dwk,
                                                                 int nq, int nk, int FP, int HP,
                                                                 int f, int hd) {
  __shared__ float red[4][64];
  const bool kv = blockIdx.y == 1;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int idx = blockIdx.x * 64 + lane;
  const int w0 = kv ? nq : 0, n = kv ? nk : nq;
  const size_t stride = (size_t)FP * HP;
  float s = 0.f;
  if (idx < f * hd) {
    const int i = idx / hd, c = idx % hd;
    const float* p = part + (size_t)w0 * stride + (size_t)i * HP + c;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    int w = wave;
    for (; w + 28 < n; w += 32) {
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] += p[(size_t)(w + 4 * j) * stride];
    }
    for (int j = 0; w < n; w += 4, ++j) acc[j & 7] += p[(size_t)w * stride];
    s = ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
  }
  red[wave][lane] = s;
  __syncthreads();
  if (wave == 0 && idx < f * hd)
    (kv ? dwk : dwq)[idx] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
}

// ---------------------------------------------------------------------------
// epilogue: out[b, l, h*hd + d] = y_gla[b, h, l, d] + alpha * y_swa[b, h, l, d]
// ---------------------------------------------------------------------------
template <typename TO>
__global__ __launch_bounds__(256) void combine_fwd_kernel(const bf16* __restrict__ yg,
                                                          const bf16* __restrict__ ys,
                                                          const float* __restrict__ alpha,
                                                          TO* __restrict__ out, int H, int L,
                                                          int hd, long n8) {
  // product and sum rounded separately, as torch's two ops: no fused multiply-add
#pragma clang fp contract(off)
  const float al = *alpha;
  const int c8 = hd / 8;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n8; i += (long)gridDim.x * 256) {
    // i enumerates output chunks in (b, l, h, d/8) order
    const int d = 8 * (int)(i % c8);
    const long blh = i / c8;
    const int hh = (int)(blh % H);
    const long bl = blh / H;
    const long b = bl / L, l = bl % L;
    const long src = ((b * H + hh) * L + l) * hd + d;
    const bf16x8 g = *reinterpret_cast<const bf16x8*>(yg + src);
    const bf16x8 s = *reinterpret_cast<const bf16x8*>(ys + src);
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = to_f32(g[e]) + al * to_f32(s[e]);
    TO* dst = out + i * 8;
    if constexpr (sizeof(TO) == 2) {
      *reinterpret_cast<bf16x8*>(dst) = to_bf8(v);
    } else {
      *reinterpret_cast<f32x4*>(dst) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{v[4], v[5], v[6], v[7]};
    }
  }
}

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float s = red[0] + red[1] + red[2] + red[3];
  __syncthreads();
  return s;
}

// d y_gla = bf16(dout), d y_swa = bf16(alpha dout), partial sums of dout * y_swa
template <typename TO>
__global__ __launch_bounds__(256) void combine_bwd_kernel(const TO* __restrict__ dout,
                                                          const bf16* __restrict__ ys,
                                                          const float* __restrict__ alpha,
                                                          bf16* __restrict__ dyg,
                                                          bf16* __restrict__ dys,
                                                          float* __restrict__ part, int H,
                                                          int L, int hd, long n8) {
  __shared__ float red[4];
  const float al = *alpha;
  const int c8 = hd / 8;
  float acc = 0.f;
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n8; i += (long)gridDim.x * 256) {
    const int d = 8 * (int)(i % c8);
    const long blh = i / c8;
    const int hh = (int)(blh % H);
    const long bl = blh / H;
    const long b = bl / L, l = bl % L;
    const long dst = ((b * H + hh) * L + l) * hd + d;
    float g[8];
    load8f(dout + i * 8, g);
    const bf16x8 s = *reinterpret_cast<const bf16x8*>(ys + dst);
    bf16x8 og, os;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      og[e] = to_bf16(g[e]);
      os[e] = to_bf16(al * g[e]);
      acc += g[e] * to_f32(s[e]);
    }
    *reinterpret_cast<bf16x8*>(dyg + dst) = og;
    *reinterpret_cast<bf16x8*>(dys + dst) = os;
  }
  const float s = block_sum(acc, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

__global__ __launch_bounds__(256) void combine_alpha_reduce_kernel(const float* __restrict__ part,
                                                                   int n, float* __restrict__ out) {
  __shared__ float red[4];
  float acc = 0.f;
  for (int i = threadIdx.x; i < n; i += 256) acc += part[i];
  const float s = block_sum(acc, red);
  if (threadIdx.x == 0) *out = s;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
static long ceil_div(long a, long b) { return (a + b - 1) / b; }

// head_dim 32, 64 or 128; feature_dim a multiple of 4 up to 128, and up to 64
// with head_dim 128 when the inputs are fp32 (bf16 inputs take 128 there too).
bool prologue_dims_supported(int hd, int f, bool bf16_in) {
  return (hd == 32 || hd == 64 || hd == 128) && f > 0 && f % 4 == 0 &&
         f <= (hd == 128 && !bf16_in ? 64 : 128);
}

static int feature_tiles(int f) { return f <= 32 ? 1 : (f <= 64 ? 2 : 4); }

// Backward: 128-row blocks of each role, and the grid (at most
// PRO_BWD_WG_PER_CU workgroups per CU on the device's CUs, no more than blocks).
static void prologue_bwd_blocks(int B, int L, int H, int Hkv, int* nbq, int* nbk) {
  *nbq = (int)ceil_div((long)B * L * H, PRO_BLOCK);
  *nbk = (int)ceil_div((long)B * L * Hkv, PRO_BLOCK);
}

static int prologue_bwd_grid(int nbq, int nbk, int occ) {
  return (int)std::min<long>((long)nbq + nbk, (long)device_geom().cus * occ);
}

size_t prologue_bwd_workspace(int B, int L, int H, int Hkv, int hd, int f) {
  int nbq, nbk;
  prologue_bwd_blocks(B, L, H, Hkv, &nbq, &nbk);
  // a q and a kv partial per workgroup, for the largest grid any instantiation uses
  return (size_t)2 * prologue_bwd_grid(nbq, nbk, PRO_BWD_WG_PER_CU) *
         (32 * feature_tiles(f)) * hd * sizeof(float);
}

template <typename T, int FT, int HT>
static hipError_t launch_fwd_t(const ProFwdArgs& a, int nq, int nk, hipStream_t st) {
  using C = Pro<T, FT, HT>;
  hipError_t e;
  if (a.f == C::FP) {
    if ((e = ensure_lds<prologue_fwd_kernel<T, FT, HT, false>>(C::FWD_LDS)) != hipSuccess) return e;
    hipLaunchKernelGGL((prologue_fwd_kernel<T, FT, HT, false>), dim3(nq + nk), dim3(256),
                       C::FWD_LDS, st, a);
  } else {
    if ((e = ensure_lds<prologue_fwd_kernel<T, FT, HT, true>>(C::FWD_LDS)) != hipSuccess) return e;
    hipLaunchKernelGGL((prologue_fwd_kernel<T, FT, HT, true>), dim3(nq + nk), dim3(256),
                       C::FWD_LDS, st, a);
  }
  return hipGetLastError();
}

template <typename T, int FT, int HT>
static hipError_t launch_bwd_t(const ProBwdArgs& a, float* dwq, float* dwk, hipStream_t st) {
  using C = ProBwd<T, FT, HT>;
  static_assert(C::FITS, "LDS budget");
  static_assert(C::OCC <= PRO_BWD_WG_PER_CU, "workspace sized for fewer workgroups");
  const int grid = prologue_bwd_grid(a.nbq, a.nbk, C::OCC);
  hipError_t e;
  if (a.f == C::FP) {
    e = ensure_lds<prologue_bwd_kernel<T, FT, HT, false>>(C::LDS);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((prologue_bwd_kernel<T, FT, HT, false>), dim3(grid), dim3(C::NT), C::LDS,
                       st, a);
  } else {
    e = ensure_lds<prologue_bwd_kernel<T, FT, HT, true>>(C::LDS);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((prologue_bwd_kernel<T, FT, HT, true>), dim3(grid), dim3(C::NT), C::LDS,
                       st, a);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  // partials: [q: grid][kv: grid] workgroups
  hipLaunchKernelGGL(prologue_dw_reduce_kernel, dim3((unsigned)ceil_div((long)a.f * a.hd, 64), 2),
                     dim3(256), 0, st, a.part, dwq, dwk, grid, grid, C::FP, C::HP, a.f, a.hd);
  return hipGetLastError();
}

template <typename T, template <typename, int, int> class Launch, typename... Args>
static hipError_t dispatch_shape(int hd, int f, Args&&... args) {
  const int ft = feature_tiles(f);
#define LZ_PRO_CASE(FT_, HD_)                                   \
  if (ft == FT_ && hd == HD_) return Launch<T, FT_, HD_ / 32>::run(args...);
  LZ_PRO_CASE(1, 32) LZ_PRO_CASE(1, 64) LZ_PRO_CASE(1, 128)
  LZ_PRO_CASE(2, 32) LZ_PRO_CASE(2, 64) LZ_PRO_CASE(2, 128)
  LZ_PRO_CASE(4, 32) LZ_PRO_CASE(4, 64)
  // head_dim 128 with more than 64 features: bf16 only (the fp32 hi/lo
  // operands double the backward's W and x tiles past the LDS)
  if constexpr (sizeof(T) == 2)
    if (ft == 4 && hd == 128) return Launch<T, 4, 4>::run(args...);
#undef LZ_PRO_CASE
  return hipErrorInvalidValue;
}

template <typename T, int FT, int HT>
struct FwdLaunch {
  static hipError_t run(const ProFwdArgs& a, int nq, int nk, hipStream_t st) {
    return launch_fwd_t<T, FT, HT>(a, nq, nk, st);
  }
};

template <typename T, int FT, int HT>
struct BwdLaunch {
  static hipError_t run(const ProBwdArgs& a, float* dwq, float* dwk, hipStream_t st) {
    return launch_bwd_t<T, FT, HT>(a, dwq, dwk, st);
  }
};

hipError_t launch_prologue_fwd(const void* q, const void* k, const void* v, const void* wq,
                               const void* wk, const void* cos, const void* sin, void* fq,
                               void* fk, void* qr, void* kr, void* vo, bool bf16_in, int B, int L,
                               int H, int Hkv, int hd, int f, int cos_bstride, hipStream_t st) {
  // one workgroup per 128-row block, up to two per CU and role when the q rows
  // write their feature maps and one without them (grid-stride beyond).
  // Measured at config 5 against 1, 1.5, 2, 2.5, 4, 8 and 16 per CU and role:
  // 155 us with fq at 2 (159 at 4, 164 at 1), 75 us without at 1 (80 at 2, 90 at 4).
  const long per_role = (long)device_geom().cus * (fq != nullptr ? 2 : 1);
  const int nq = (int)std::min<long>(ceil_div((long)B * L * H, PRO_BLOCK), per_role);
  const int nk = (int)std::min<long>(ceil_div((long)B * L * Hkv, PRO_BLOCK), per_role);
  ProFwdArgs a{q, k, v, wq, wk, cos, sin,
               static_cast<bf16*>(fq), static_cast<bf16*>(fk), static_cast<bf16*>(qr),
               static_cast<bf16*>(kr), static_cast<bf16*>(vo),
               B, L, H, Hkv, hd, f, cos_bstride, nq};
  return bf16_in ? dispatch_shape<bf16, FwdLaunch>(hd, f, a, nq, nk, st)
                 : dispatch_shape<float, FwdLaunch>(hd, f, a, nq, nk, st);
}

hipError_t launch_prologue_bwd(const void* q, const void* k, const void* wq, const void* wk,
                               const void* cos, const void* sin, const void* dfq,
                               const void* dfk, const void* dqr, const void* dkr,
                               const void* dv, const void* dv2, void* dq, void* dk, void* dvo,
                               float* dwq, float* dwk, bool bf16_in, int B, int L, int H, int Hkv,
                               int hd, int f, int cos_bstride, float* ws, hipStream_t st) {
  int nbq, nbk;
  prologue_bwd_blocks(B, L, H, Hkv, &nbq, &nbk);
  ProBwdArgs a{q, k, wq, wk, cos, sin, static_cast<const bf16*>(dfq),
               static_cast<const bf16*>(dfk), static_cast<const bf16*>(dqr),
               static_cast<const bf16*>(dkr), static_cast<const bf16*>(dv),
               static_cast<const bf16*>(dv2), dq, dk, dvo, ws,
               B, L, H, Hkv, hd, f, cos_bstride, nbq, nbk};
  return bf16_in ? dispatch_shape<bf16, BwdLaunch>(hd, f, a, dwq, dwk, st)
                 : dispatch_shape<float, BwdLaunch>(hd, f, a, dwq, dwk, st);
}

size_t combine_bwd_workspace() { return CMB_BLOCKS * sizeof(float); }

static int combine_blocks(long n8) { return (int)std::min<long>(ceil_div(n8, 256), CMB_BLOCKS); }

hipError_t launch_combine_fwd(const void* yg, const void* ys, const float* alpha, void* out,
                              bool bf16_out, int B, int H, int L, int hd, hipStream_t st) {
  const long n8 = (long)B * H * L * hd / 8;
  const int grid = (int)std::min<long>(ceil_div(n8, 256), 8192);
  if (bf16_out)
    hipLaunchKernelGGL(combine_fwd_kernel<bf16>, dim3(grid), dim3(256), 0, st,
                       static_cast<const bf16*>(yg), static_cast<const bf16*>(ys), alpha,
                       static_cast<bf16*>(out), H, L, hd, n8);
  else
    hipLaunchKernelGGL(combine_fwd_kernel<float>, dim3(grid), dim3(256), 0, st,
                       static_cast<const bf16*>(yg), static_cast<const bf16*>(ys), alpha,
                       static_cast<float*>(out), H, L, hd, n8);
  return hipGetLastError();
}

hipError_t launch_combine_bwd(const void* dout, const void* ys, const float* alpha, void* dyg,
                              void* dys, float* dalpha, bool bf16_out, int B, int H, int L,
                              int hd, float* ws, hipStream_t st) {
  const long n8 = (long)B * H * L * hd / 8;
  const int grid = combine_blocks(n8);
  if (bf16_out)
    hipLaunchKernelGGL(combine_bwd_kernel<bf16>, dim3(grid), dim3(256), 0, st,
                       static_cast<const bf16*>(dout), static_cast<const bf16*>(ys), alpha,
                       static_cast<bf16*>(dyg), static_cast<bf16*>(dys), ws, H, L, hd, n8);
  else
    hipLaunchKernelGGL(combine_bwd_kernel<float>, dim3(grid), dim3(256), 0, st,
                       static_cast<const float*>(dout), static_cast<const bf16*>(ys), alpha,
                       static_cast<bf16*>(dyg), static_cast<bf16*>(dys), ws, H, L, hd, n8);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(combine_alpha_reduce_kernel, dim3(1), dim3(256), 0, st, ws, grid, dalpha);
  return hipGetLastError();
}

}  // namespace lz
