// Prologue and epilogue of the LizardAttention layer (src/lizard_attention.py:
// 78-97): everything between the q/k/v projections and o_proj except the two
// attention branches.
//
// Prologue, per token row of the projections ([B, L, heads, hd] row-major,
// rows ordered (b, l, head)):
//   fq = [softmax(q Wq^T), softmax(-q Wq^T)]      (Hedgehog, :9-11, F = 2f)
//   qr = rope(q)                                  (rotate_half RoPE, :88)
//   fk, kr, v likewise from the kv heads, each written to the H / Hkv query
//   heads of its group (the repeat_interleave of :73-76)
// all in fp32 from the inputs' values, written once as the bf16 [B, H, L, .]
// operands of the GLA and SWA kernels.  x W^T is a bf16 MFMA product; fp32
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
constexpr int PRO_WG_PER_ROLE = 256;              // backward workgroups per role (q, kv)
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
  static constexpr int DP = lds_pitch(FP);      // backward dxw tile [128][DP]
  static constexpr int QP = lds_pitch(HP);      // backward x tile [128][QP] (per part)
  static constexpr int BWD_LDS =
      (PARTS * W_ELEMS + PRO_BLOCK * DP + PARTS * PRO_BLOCK * QP) * 2;
  static_assert(BWD_LDS <= 160 * 1024 && FWD_LDS <= 160 * 1024, "LDS budget");
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
  int B, L, H, Hkv, hd, f, cos_bstride, nq_wg;
};

// W [f][hd] (type T) into LDS as bf16 hi (and lo) tiles [FP][WP], zero rows
// beyond f.
template <typename T, int FT, int HT>
__device__ void load_weight(const T* __restrict__ w, int f, bf16* hi, bf16* lo) {
  using C = Pro<T, FT, HT>;
  for (int i = threadIdx.x; i < C::FP * C::HP; i += 256) {
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

// Row statistics of the two softmaxes over the valid features (< f):
// maxima and reciprocal sums, combined over both lane halves.
template <typename T, int FT, int HT>
__device__ __forceinline__ void softmax_stats(const bf16x8 (&xh)[Pro<T, FT, HT>::HK],
                                              const bf16x8 (&xl)[Pro<T, FT, HT>::HK],
                                              const bf16* w_hi, const bf16* w_lo, int f,
                                              int lane, float& mp, float& mn, float& ip,
                                              float& in) {
  const int h = lane >> 5;
  mp = NEG_INF;
  mn = NEG_INF;
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const f32x16 acc = project_tile<T, FT, HT>(ft, xh, xl, w_hi, w_lo, lane);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (32 * ft + acc_row(r, h) < f) {
        mp = fmaxf(mp, acc[r]);
        mn = fmaxf(mn, -acc[r]);
      }
  }
  mp = fmaxf(mp, xhalf(mp));
  mn = fmaxf(mn, xhalf(mn));
  float sp = 0.f, sn = 0.f;
#pragma unroll
  for (int ft = 0; ft < FT; ++ft) {
    const f32x16 acc = project_tile<T, FT, HT>(ft, xh, xl, w_hi, w_lo, lane);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      if (32 * ft + acc_row(r, h) < f) {
        sp += fexp(acc[r] - mp);
        sn += fexp(-acc[r] - mn);
      }
  }
  sp += xhalf(sp);
  sn += xhalf(sn);
  ip = 1.f / sp;
  in = 1.f / sn;
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
// ([32][pitch] bf16), to the rows' output heads in chunks of CH elements.
// Row r's output base row (the obase of lane r, split in two ints) comes
// from lane r by a cross-lane read.
template <int CH>
__device__ __forceinline__ void copy_rows(const bf16* stage, int pitch, bf16* __restrict__ out,
                                          int ob_lo, int ob_hi, int row0, int nrows, int f,
                                          int half, int group, int L, int lane) {
  typedef __bf16 chunk_t __attribute__((ext_vector_type(CH)));
  const int cpr = f / CH;
  for (int i = lane; i < PRO_ROWS * cpr; i += 64) {
    const int r = i / cpr, c = CH * (i - r * cpr);
    const long base = ((long)__shfl(ob_hi, r) << 32) | (unsigned)__shfl(ob_lo, r);
    if (row0 + r >= nrows) continue;
    const chunk_t val = *reinterpret_cast<const chunk_t*>(stage + r * pitch + c);
    for (int g = 0; g < group; ++g)
      *reinterpret_cast<chunk_t*>(out + (base + (long)g * L) * (2 * f) + half * f + c) = val;
  }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <typename T, int FT, int HT>
__global__ __launch_bounds__(256) void prologue_fwd_kernel(ProFwdArgs a) {
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
  const int group = kv ? a.H / a.Hkv : 1;
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
    // [B, H, L, .] row of this row's first output head; the group's next heads
    // are L rows apart
    const long obase = ((long)pos.b * a.H + pos.head * group) * a.L + pos.l;

    bf16x8 xh[C::HK], xl[C::HK];
    {
      float xf[C::HK][8];
#pragma unroll
      for (int kb = 0; kb < C::HK; ++kb) {
        if (live) {
          load8f(x + (long)row * hd + 16 * kb + 8 * h, xf[kb]);
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) xf[kb][e] = 0.f;
        }
      }
      // RoPE (and the kv heads' v) from the fp32 row values: column
      // m = 16 kb + 8 h + e pairs with m + hd/2, the same column of kb + HK/2
      if (live) {
        const long tab = ((long)pos.b * a.cos_bstride + pos.l) * hd;
#pragma unroll
        for (int kb = 0; kb < C::HK / 2; ++kb) {
          const int kb2 = kb + C::HK / 2;
          float c1[8], s1[8], c2[8], s2[8];
          load8f(cs + tab + 16 * kb + 8 * h, c1);
          load8f(sn + tab + 16 * kb + 8 * h, s1);
          load8f(cs + tab + 16 * kb2 + 8 * h, c2);
          load8f(sn + tab + 16 * kb2 + 8 * h, s2);
          bf16x8 o1, o2;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            o1[e] = to_bf16(xf[kb][e] * c1[e] - xf[kb2][e] * s1[e]);
            o2[e] = to_bf16(xf[kb2][e] * c2[e] + xf[kb][e] * s2[e]);
          }
          for (int g = 0; g < group; ++g) {
            bf16* dst = rout + (obase + (long)g * a.L) * hd;
            *reinterpret_cast<bf16x8*>(dst + 16 * kb + 8 * h) = o1;
            *reinterpret_cast<bf16x8*>(dst + 16 * kb2 + 8 * h) = o2;
          }
        }
        if (kv) {
          const T* vrow = static_cast<const T*>(a.v) + (long)row * hd;
#pragma unroll
          for (int kb = 0; kb < C::HK; ++kb) {
            float vf[8];
            load8f(vrow + 16 * kb + 8 * h, vf);
            const bf16x8 o = to_bf8(vf);
            for (int g = 0; g < group; ++g)
              *reinterpret_cast<bf16x8*>(a.vo + (obase + (long)g * a.L) * hd + 16 * kb + 8 * h) =
                  o;
          }
        }
      }
#pragma unroll
      for (int kb = 0; kb < C::HK; ++kb) {
        xh[kb] = to_bf8(xf[kb]);
        if constexpr (C::SPLIT) xl[kb] = low8(xf[kb], xh[kb]);
      }
    }
    float mp, mn, ip, in;
    softmax_stats<T, FT, HT>(xh, xl, w_hi, w_lo, f, lane, mp, mn, ip, in);

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
            o[e] = to_bf16(half == 0 ? fexp(s - mp) * ip : fexp(-s - mn) * in);
          }
          *reinterpret_cast<bf16x4*>(stage + (lane & 31) * C::SP + 32 * ft + 8 * q4 + 4 * h) = o;
        }
      }
      wave_sync();
      if (f % 8 == 0)
        copy_rows<8>(stage, C::SP, fout, ob_lo, ob_hi, row0, nrows, f, half, group, a.L, lane);
      else
        copy_rows<4>(stage, C::SP, fout, ob_lo, ob_hi, row0, nrows, f, half, group, a.L, lane);
      wave_sync();
    }
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
template <typename T, int FT, int HT>
__global__ __launch_bounds__(256) void prologue_bwd_kernel(ProBwdArgs a) {
  using C = Pro<T, FT, HT>;
  constexpr int TILES = FT * HT;
  constexpr int OWN = (TILES + PRO_WAVES - 1) / PRO_WAVES;   // dW tiles per wave
  extern __shared__ __attribute__((aligned(16))) char smem[];
  bf16* w_hi = reinterpret_cast<bf16*>(smem);
  bf16* w_lo = w_hi + C::W_ELEMS;
  bf16* d_l = w_hi + C::PARTS * C::W_ELEMS;          // dxw tile [128][DP]
  bf16* x_hi = d_l + PRO_BLOCK * C::DP;              // x tile [128][QP]
  bf16* x_lo = x_hi + PRO_BLOCK * C::QP;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, h = lane >> 5;
  const int lrow = wave * PRO_ROWS + (lane & 31);    // this lane's row in the LDS tiles

  const bool kv = (int)blockIdx.x >= a.nq_wg;
  const int wg = kv ? blockIdx.x - a.nq_wg : blockIdx.x;
  const int nwg = kv ? gridDim.x - a.nq_wg : a.nq_wg;
  const int heads_in = kv ? a.Hkv : a.H;
  const int group = kv ? a.H / a.Hkv : 1;
  const int nrows = a.B * a.L * heads_in;
  const T* x = static_cast<const T*>(kv ? a.k : a.q);
  const bf16* dphi = kv ? a.dfk : a.dfq;
  const bf16* drope = kv ? a.dkr : a.dqr;
  T* dx = static_cast<T*>(kv ? a.dk : a.dq);
  const T* cs = static_cast<const T*>(a.cos);
  const T* sn = static_cast<const T*>(a.sin);
  const int f = a.f, hd = C::HP, half_hd = C::HP / 2, F2 = 2 * a.f;

  load_weight<T, FT, HT>(static_cast<const T*>(kv ? a.wk : a.wq), f, w_hi, w_lo);

  f32x16 dw[OWN];
#pragma unroll
  for (int i = 0; i < OWN; ++i) dw[i] = zero16();

  for (int blk = wg; blk * PRO_BLOCK < nrows; blk += nwg) {
    const int row = blk * PRO_BLOCK + lrow;
    const bool live = row < nrows;
    const RowPos pos = decode(live ? row : 0, a.L, heads_in);
    // [B, H, L, .] row of this row's first head; the group's heads are L rows apart
    const long obase = ((long)pos.b * a.H + pos.head * group) * a.L + pos.l;

    bf16x8 xh[C::HK], xl[C::HK];
#pragma unroll
    for (int kb = 0; kb < C::HK; ++kb) {
      float xf[8];
      if (live) {
        load8f(x + (long)row * hd + 16 * kb + 8 * h, xf);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xf[e] = 0.f;
      }
      xh[kb] = to_bf8(xf);
      *reinterpret_cast<bf16x8*>(x_hi + lrow * C::QP + 16 * kb + 8 * h) = xh[kb];
      if constexpr (C::SPLIT) {
        xl[kb] = low8(xf, xh[kb]);
        *reinterpret_cast<bf16x8*>(x_lo + lrow * C::QP + 16 * kb + 8 * h) = xl[kb];
      }
    }
    __syncthreads();   // W tiles (first pass) and nothing else pending
    float mp, mn, ip, in;
    softmax_stats<T, FT, HT>(xh, xl, w_hi, w_lo, f, lane, mp, mn, ip, in);

    // u = p dp - n dn per feature; s_p = <p, dp>, s_n = <n, dn>
    f32x16 dxw[FT];
    float s_p = 0.f, s_n = 0.f;
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) {
      f32x4 dp[4], dn[4];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int c = 32 * ft + 8 * q4 + 4 * h;
        dp[q4] = f32x4{0.f, 0.f, 0.f, 0.f};
        dn[q4] = dp[q4];
        if (live && c < f) {
          for (int g = 0; g < group; ++g) {
            const bf16* src = dphi + (obase + (long)g * a.L) * F2;
            dp[q4] += load4f(src + c);
            dn[q4] += load4f(src + f + c);
          }
        }
      }
      const f32x16 acc = project_tile<T, FT, HT>(ft, xh, xl, w_hi, w_lo, lane);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float u = 0.f;
        if (32 * ft + acc_row(r, h) < f) {
          const float p = fexp(acc[r] - mp) * ip;
          const float n = fexp(-acc[r] - mn) * in;
          const float pd = p * dp[r >> 2][r & 3], nd = n * dn[r >> 2][r & 3];
          u = pd - nd;
          s_p += pd;
          s_n += nd;
        }
        dxw[ft][r] = u;
      }
    }
    s_p += xhalf(s_p);
    s_n += xhalf(s_n);
#pragma unroll
    for (int ft = 0; ft < FT; ++ft) {
      const f32x16 acc = project_tile<T, FT, HT>(ft, xh, xl, w_hi, w_lo, lane);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (32 * ft + acc_row(r, h) < f) {
          const float p = fexp(acc[r] - mp) * ip;
          const float n = fexp(-acc[r] - mn) * in;
          dxw[ft][r] += n * s_n - p * s_p;
        }
    }

    // dx_phi^T = W^T dxw^T: hd rows (registers), this wave's rows (lanes)
    f32x16 dacc[HT];
#pragma unroll
    for (int ht = 0; ht < HT; ++ht) {
      dacc[ht] = zero16();
#pragma unroll
      for (int ft = 0; ft < FT; ++ft)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const bf16x8 w = tr_operand(w_hi, C::WP, 32 * ft + 16 * kb, 32 * ht, lane);
          const bf16x8 dh = acc_operand(dxw[ft], kb);
          dacc[ht] = mfma(w, dh, dacc[ht]);
          dacc[ht] = mfma(w, acc_operand_lo(dxw[ft], kb), dacc[ht]);
          if constexpr (C::SPLIT)
            dacc[ht] = mfma(tr_operand(w_lo, C::WP, 32 * ft + 16 * kb, 32 * ht, lane), dh,
                            dacc[ht]);
        }
    }

    // dxw hi into the LDS tile now, lo kept as bf16 until the tile is free:
    // the fp32 dxw dies here
    bf16x4 dlo[FT][4];
#pragma unroll
    for (int ft = 0; ft < FT; ++ft)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        bf16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float v = dxw[ft][4 * q4 + e];
          o[e] = to_bf16(v);
          dlo[ft][q4][e] = to_bf16(v - to_f32(o[e]));
        }
        *reinterpret_cast<bf16x4*>(d_l + lrow * C::DP + 32 * ft + 8 * q4 + 4 * h) = o;
      }

    // dx = dx_phi + rope^T(drope): dx[m] = dr[m] cos[m] + dr[m + hd/2] sin[m + hd/2]
    // for m < hd/2, dr[m] cos[m] - dr[m - hd/2] sin[m - hd/2] otherwise
    // (drope summed over the group's heads); the kv rows also sum dv.
    if (live) {
      const long tab = ((long)pos.b * a.cos_bstride + pos.l) * hd;
#pragma unroll
      for (int ht = 0; ht < HT; ++ht)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const int m = 32 * ht + 8 * q4 + 4 * h;
          const int mp2 = m < half_hd ? m + half_hd : m - half_hd;
          const float sign = m < half_hd ? 1.f : -1.f;
          f32x4 dr = {0.f, 0.f, 0.f, 0.f}, dr2 = dr, dvs = dr;
          for (int g = 0; g < group; ++g) {
            const long o = (obase + (long)g * a.L) * hd;
            dr += load4f(drope + o + m);
            dr2 += load4f(drope + o + mp2);
            if (kv) {
              dvs += load4f(a.dv + o + m);
              if (a.dv2) dvs += load4f(a.dv2 + o + m);
            }
          }
          const f32x4 c = load4f(cs + tab + m), s2 = load4f(sn + tab + mp2);
          f32x4 out;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            out[e] = dacc[ht][4 * q4 + e] + dr[e] * c[e] + sign * dr2[e] * s2[e];
          store4v(dx + (long)row * hd + m, out);
          if (kv) store4v(static_cast<T*>(a.dvo) + (long)row * hd + m, dvs);
        }
    }

    // dW += dxw^T x over the workgroup's 128 rows: dxw hi, then lo, through LDS
#pragma unroll
    for (int part = 0; part < 2; ++part) {
      if (part == 1) {
#pragma unroll
        for (int ft = 0; ft < FT; ++ft)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            *reinterpret_cast<bf16x4*>(d_l + lrow * C::DP + 32 * ft + 8 * q4 + 4 * h) =
                dlo[ft][q4];
      }
      __syncthreads();
#pragma unroll
      for (int i = 0; i < OWN; ++i) {
        const int t = wave + PRO_WAVES * i;
        if (t < TILES) {
          const int ft = t / HT, ht = t % HT;
#pragma unroll
          for (int ks = 0; ks < PRO_BLOCK / 16; ++ks) {
            const bf16x8 d = tr_operand(d_l, C::DP, 16 * ks, 32 * ft, lane);
            dw[i] = mfma(d, tr_operand(x_hi, C::QP, 16 * ks, 32 * ht, lane), dw[i]);
            if (C::SPLIT && part == 0)
              dw[i] = mfma(d, tr_operand(x_lo, C::QP, 16 * ks, 32 * ht, lane), dw[i]);
          }
        }
      }
      __syncthreads();
    }
  }

  // this workgroup's partial dW [FP][HP]: lane = column, registers = rows
  float* part = a.part + (size_t)blockIdx.x * C::FP * C::HP;
#pragma unroll
  for (int i = 0; i < OWN; ++i) {
    const int t = wave + PRO_WAVES * i;
    if (t < TILES) {
      const int ft = t / HT, ht = t % HT;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        part[(32 * ft + acc_row(r, h)) * C::HP + 32 * ht + (lane & 31)] = dw[i][r];
    }
  }
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
// with head_dim 128 (the GLA kernels take F = 2 feature_dim <= 128 when D = 128).
bool prologue_dims_supported(int hd, int f) {
  return (hd == 32 || hd == 64 || hd == 128) && f > 0 && f % 4 == 0 &&
         f <= (hd == 128 ? 64 : 128);
}

static int feature_tiles(int f) { return f <= 32 ? 1 : (f <= 64 ? 2 : 4); }

void prologue_grid(int B, int L, int H, int Hkv, int* nq, int* nk) {
  const long rq = (long)B * L * H, rk = (long)B * L * Hkv;
  *nq = (int)std::min<long>(ceil_div(rq, PRO_BLOCK), PRO_WG_PER_ROLE);
  *nk = (int)std::min<long>(ceil_div(rk, PRO_BLOCK), PRO_WG_PER_ROLE);
}

size_t prologue_bwd_workspace(int B, int L, int H, int Hkv, int hd, int f) {
  int nq, nk;
  prologue_grid(B, L, H, Hkv, &nq, &nk);
  return (size_t)(nq + nk) * (32 * feature_tiles(f)) * hd * sizeof(float);
}

template <typename T, int FT, int HT>
static hipError_t launch_fwd_t(const ProFwdArgs& a, int nq, int nk, hipStream_t st) {
  using C = Pro<T, FT, HT>;
  hipError_t e = ensure_lds<prologue_fwd_kernel<T, FT, HT>>(C::FWD_LDS);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((prologue_fwd_kernel<T, FT, HT>), dim3(nq + nk), dim3(256), C::FWD_LDS, st,
                     a);
  return hipGetLastError();
}

template <typename T, int FT, int HT>
static hipError_t launch_bwd_t(const ProBwdArgs& a, float* dwq, float* dwk, int nq, int nk,
                               hipStream_t st) {
  using C = Pro<T, FT, HT>;
  hipError_t e = ensure_lds<prologue_bwd_kernel<T, FT, HT>>(C::BWD_LDS);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((prologue_bwd_kernel<T, FT, HT>), dim3(nq + nk), dim3(256), C::BWD_LDS, st,
                     a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(prologue_dw_reduce_kernel, dim3((unsigned)ceil_div((long)a.f * a.hd, 64), 2),
                     dim3(256), 0, st, a.part, dwq, dwk, nq, nk, C::FP, C::HP, a.f, a.hd);
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
  static hipError_t run(const ProBwdArgs& a, float* dwq, float* dwk, int nq, int nk,
                        hipStream_t st) {
    return launch_bwd_t<T, FT, HT>(a, dwq, dwk, nq, nk, st);
  }
};

hipError_t launch_prologue_fwd(const void* q, const void* k, const void* v, const void* wq,
                               const void* wk, const void* cos, const void* sin, void* fq,
                               void* fk, void* qr, void* kr, void* vo, bool bf16_in, int B, int L,
                               int H, int Hkv, int hd, int f, int cos_bstride, hipStream_t st) {
  int nq, nk;
  prologue_grid(B, L, H, Hkv, &nq, &nk);
  // the forward needs no partials: one workgroup per 128-row block, up to 4x the backward's
  nq = (int)std::min<long>(ceil_div((long)B * L * H, PRO_BLOCK), 4 * PRO_WG_PER_ROLE);
  nk = (int)std::min<long>(ceil_div((long)B * L * Hkv, PRO_BLOCK), 4 * PRO_WG_PER_ROLE);
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
  int nq, nk;
  prologue_grid(B, L, H, Hkv, &nq, &nk);
  ProBwdArgs a{q, k, wq, wk, cos, sin, static_cast<const bf16*>(dfq),
               static_cast<const bf16*>(dfk), static_cast<const bf16*>(dqr),
               static_cast<const bf16*>(dkr), static_cast<const bf16*>(dv),
               static_cast<const bf16*>(dv2), dq, dk, dvo, ws,
               B, L, H, Hkv, hd, f, cos_bstride, nq};
  return bf16_in ? dispatch_shape<bf16, BwdLaunch>(hd, f, a, dwq, dwk, nq, nk, st)
                 : dispatch_shape<float, BwdLaunch>(hd, f, a, dwq, dwk, nq, nk, st);
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
