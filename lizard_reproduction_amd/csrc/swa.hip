// Sliding-window softmax attention with learned sink logits, forward and
// backward, for gfx950.
//
// Math (reference: src/lizard_attention.py:34-44 dense form; operator API
// src/kernels/swa.py:136-183):
//   s_it = q_i . k_t / sqrt(d) for keys i-W < t <= i (t < L)
//   y_i  = sum_t e^{s_it} v_t / (sum_j e^{meta_j} + sum_t e^{s_it})
//   lse_i = log(sum_j e^{meta_j} + sum_t e^{s_it})
// Backward, with p_it = e^{s_it - lse_i}:
//   delta_i = dy_i . y_i = sum_t p_it (dy_i . v_t)     (the sinks carry no value)
//   ds_it = p_it (dy_i . v_t - delta_i)
//   dq_i = scale sum_t ds_it k_t,  dk_t = scale sum_i ds_it q_i,
//   dv_t = sum_i p_it dy_i,  dmeta_j = -sum_i e^{meta_j - lse_i} delta_i
// The reference forms delta from the bf16 output (src/kernels/swa.py:164);
// here it is the fp32 sum above, taken from the same p and dy.v the backward
// computes anyway, so nothing beyond y and lse is saved by the forward.
//
// Layout: q, k, v, y, dy, dq, dk, dv are [BH, L, d] row-major; lse, delta
// [BH, L] fp32.  A workgroup is 4 waves and covers 128 rows of its own side
// (queries in the forward and dq kernels, keys in the dk/dv kernel), 32 per
// wave, held in registers as MFMA operands; the other side streams through
// LDS in 64-row row-major tiles, the next tile prefetched into registers.
// Operands that contract over rows of a staged tile (V^T, K^T, Q^T, dY^T)
// come from LDS transpose reads.  Scores are computed with the staged side as
// the MFMA A operand, so each lane owns one row of its own side and the
// softmax statistics are per-lane scalars; P and dS then feed the next product
// straight from the accumulator registers.  Consecutive workgroups of one
// (b, h) are mapped to one XCD so that the tiles they share hit one L2.
#include "common.hpp"

namespace lz {

constexpr int SWA_META_BLOCK = 64;   // sinks per pass of a block's dmeta partials
constexpr int SWA_ROWS = 128;   // own-side rows per workgroup
constexpr int SWA_TILE = 64;    // streamed rows per LDS tile

template <int DP>
struct SwaCfg {
  static constexpr int P = lds_pitch(DP);                // LDS row pitch (elements)
  static constexpr int NL = SWA_TILE * DP / 8 / 256;     // 16-byte loads per thread per tile
  static constexpr int TILE_BYTES = SWA_TILE * P * 2;
};


// rows [r0, r0+64) of a [L x d] matrix, 16 bytes per load (zero outside it)
template <int DP>
__device__ __forceinline__ void swa_load(uint4 (&reg)[SwaCfg<DP>::NL], const bf16* __restrict__ base,
                                         int r0, int L, int d, bool vec) {
  load_items<DP, 256, SwaCfg<DP>::NL, 256 * SwaCfg<DP>::NL>(reg, base, r0, L, d, vec);
}

template <int DP>
__device__ __forceinline__ void swa_store(const uint4 (&reg)[SwaCfg<DP>::NL], bf16* tile) {
  constexpr int K8 = DP / 8;
#pragma unroll
  for (int i = 0; i < SwaCfg<DP>::NL; ++i) {
    const int idx = threadIdx.x + 256 * i;
    *reinterpret_cast<uint4*>(tile + (idx / K8) * SwaCfg<DP>::P + (idx % K8) * 8) = reg[i];
  }
}

// The wave's own 32 rows as MFMA operands with contiguous k slots
// (columns 16 kb + 8 h .. +8 of row `row`), zero outside the matrix.
template <int DP>
__device__ __forceinline__ void own_rows(const bf16* __restrict__ base, int row, int L, int d,
                                         int h, bool vec, bf16x8 (&reg)[DP / 16]) {
#pragma unroll
  for (int kb = 0; kb < DP / 16; ++kb)
    reg[kb] = __builtin_bit_cast(bf16x8, gload8(base, row, 16 * kb + 8 * h, L, d, vec));
}

// Is key t inside the window of query i (i - W < t <= i)?  One unsigned
// compare.  The kernels need no t < L or i < L test: for a query row inside
// the sequence the window test already gives t <= i < L, a query row past L
// is never stored (and reads zero q and dy rows, so it adds exactly 0 to dk
// and dv), and a key row past L is never stored either.
__device__ __forceinline__ bool in_window(int i, int t, int W) {
  return (unsigned)(i - t) < (unsigned)W;
}

// Does key block [k0, k0+32) meet the windows of queries [q0, q0+32)?
__device__ __forceinline__ bool blocks_meet(int q0, int k0, int L, int W) {
  return q0 < L && k0 < L && k0 <= q0 + 31 && k0 + 31 >= q0 - W + 1;
}

// ----------------------------------------------------------------------------
// forward
// ----------------------------------------------------------------------------
// Workgroups per CU the forward asks the compiler to fit in registers: at
// d <= 64 four (122 VGPRs at d = 64 instead of 178 unconstrained), so four
// waves per SIMD overlap each other's loads; two at d = 128 (no spills).
template <int DP, bool VEC>
constexpr int swa_fwd_occupancy() {
  return DP <= 32 ? 4 : DP <= 64 ? (VEC ? 4 : 3) : DP <= 128 ? 2 : 1;
}

// RES: the window's key tiles (at most SWA_RES of them) are loaded at once,
// each into its own LDS slot, behind one barrier, where the streaming form
// waits for one tile per barrier: for grids of at most two workgroups per CU,
// where each workgroup's chain of tile loads, not the CU's throughput, sets
// the time.
constexpr int SWA_RES = 4;

template <int DP, bool VEC, bool RES>
__global__ __launch_bounds__(256, (RES ? 2 : swa_fwd_occupancy<DP, VEC>())) void swa_fwd_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ meta, int n_meta, bf16* __restrict__ y, float* __restrict__ lse,
    int BH, int L, int d, int W, float scale, int per, int nx, int KG) {
  using Cfg = SwaCfg<DP>;
  constexpr int P = Cfg::P;
  constexpr int NSLOT = RES ? SWA_RES : 1;
  extern __shared__ __align__(16) char smem[];
  // k tile of slot i at smem + i TILE_BYTES, v tile at smem + (NSLOT + i) TILE_BYTES
  auto kslot = [&](int i) { return reinterpret_cast<bf16*>(smem + i * Cfg::TILE_BYTES); };
  auto vslot = [&](int i) { return reinterpret_cast<bf16*>(smem + (NSLOT + i) * Cfg::TILE_BYTES); };

  const int nqb = (L + SWA_ROWS - 1) / SWA_ROWS;
  const int lb = xcd_block(blockIdx.x, per, nx);
  if (lb >= BH * nqb) return;
  const int bh = lb / nqb, Q0 = (lb % nqb) * SWA_ROWS;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 31, h = lane >> 5;
  const int q0 = Q0 + wave * 32, qi = q0 + col;
  const size_t base = (size_t)bh * L * d;
  const size_t kvbase = (size_t)(bh / KG) * L * d;   // k, v: the kv head (KG query heads share one)
  const bool vec = VEC || (d & 7) == 0;

  bf16x8 qreg[DP / 16];
  own_rows<DP>(q + base, qi, L, d, h, vec, qreg);

  // running max and sum start from the sinks (src/kernels/swa.py:34-38).  The
  // max is kept in log2 units, u = s log2(e): a score's weight is then
  // exp2(q.k c - m) with c = scale log2(e), one FMA and the hardware exp2.
  const float c = scale * LOG2E;
  float m_i = -1e30f;
  for (int j = 0; j < n_meta; ++j) m_i = fmaxf(m_i, meta[j] * LOG2E);
  float l_i = 0.f;
  for (int j = 0; j < n_meta; ++j) l_i += __builtin_amdgcn_exp2f(meta[j] * LOG2E - m_i);

  f32x16 o[DP / 32];
#pragma unroll
  for (int t = 0; t < DP / 32; ++t) o[t] = zero16();

  // the work of one key tile (keys t0 .. t0+63 in k_l, v_l)
  auto tile = [&](const bf16* k_l, const bf16* v_l, int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int k0 = t0 + 32 * half;
      if (!blocks_meet(q0, k0, L, W)) continue;
      f32x16 s = zero16();
#pragma unroll
      for (int kb = 0; kb < DP / 16; ++kb)
        s = mfma(row_operand(k_l, P, 32 * half + col, 16 * kb, h), qreg[kb], s);
      // only blocks that straddle the window's start or the diagonal are
      // masked: keys [k0, k0 + 32) lie in every window of queries
      // [q0, q0 + 32) when k0 + 31 <= q0 and k0 >= q0 + 32 - W (uniform per wave)
      float mx = NEG_INF;
      if (k0 + 31 <= q0 && k0 >= q0 + 32 - W) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          s[r] = in_window(qi, k0 + acc_row(r, h), W) ? s[r] : NEG_INF;
          mx = fmaxf(mx, s[r]);
        }
      }
      mx = fmaxf(mx, xhalf(mx));
      const float m_new = fmaxf(m_i, mx * c);
      const float alpha = __builtin_amdgcn_exp2f(m_i - m_new);
      float ps = 0.f;
      bf16x8 p[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = __builtin_amdgcn_exp2f(fmaf(s[r], c, -m_new));
        ps += e;
        p[r >> 3][r & 7] = to_bf16(e);
      }
      ps += xhalf(ps);
      l_i = l_i * alpha + ps;
      m_i = m_new;
#pragma unroll
      for (int t = 0; t < DP / 32; ++t) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          o[t] = mfma(tr_operand(v_l, P, 32 * half + 16 * kb, t * 32, lane), p[kb], o[t]);
      }
    }
  };

  const int klo = (max(0, Q0 - W + 1) / SWA_TILE) * SWA_TILE;
  const int khi = min(L, Q0 + SWA_ROWS);
  if constexpr (RES) {
    const int nt = (khi - klo + SWA_TILE - 1) / SWA_TILE;   // <= SWA_RES (the launcher's test)
    uint4 rk[SWA_RES][Cfg::NL], rv[SWA_RES][Cfg::NL];
#pragma unroll
    for (int i = 0; i < SWA_RES; ++i)
      if (i < nt) {
        swa_load<DP>(rk[i], k + kvbase, klo + i * SWA_TILE, L, d, vec);
        swa_load<DP>(rv[i], v + kvbase, klo + i * SWA_TILE, L, d, vec);
      }
#pragma unroll
    for (int i = 0; i < SWA_RES; ++i)
      if (i < nt) {
        swa_store<DP>(rk[i], kslot(i));
        swa_store<DP>(rv[i], vslot(i));
      }
    __syncthreads();
    for (int i = 0; i < nt; ++i) tile(kslot(i), vslot(i), klo + i * SWA_TILE);
  } else {
    uint4 rk[Cfg::NL], rv[Cfg::NL];
    swa_load<DP>(rk, k + kvbase, klo, L, d, vec);
    swa_load<DP>(rv, v + kvbase, klo, L, d, vec);
    swa_store<DP>(rk, kslot(0));
    swa_store<DP>(rv, vslot(0));
    __syncthreads();
    for (int t0 = klo; t0 < khi; t0 += SWA_TILE) {
      const bool more = t0 + SWA_TILE < khi;
      if (more) {
        swa_load<DP>(rk, k + kvbase, t0 + SWA_TILE, L, d, vec);
        swa_load<DP>(rv, v + kvbase, t0 + SWA_TILE, L, d, vec);
      }
      tile(kslot(0), vslot(0), t0);
      if (more) {
        __syncthreads();
        swa_store<DP>(rk, kslot(0));
        swa_store<DP>(rv, vslot(0));
        __syncthreads();
      }
    }
  }
  // every lane stores (rows past L are dropped): the row store swaps across lane halves
  const float inv = 1.f / l_i;
#pragma unroll
  for (int t = 0; t < DP / 32; ++t) store_acc_row<bf16>(y + base, qi, t * 32, L, d, vec, o[t], inv, h);
  if (qi < L && h == 0) lse[(size_t)bh * L + qi] = m_i * LN2 + flog(l_i);
}

// Workgroups per CU the backward kernels ask the compiler to fit in
// registers (VGPRs and AGPRs together): three at d <= 32, two at d <= 64
// (about 200 VGPRs, no spills), one beyond, where two would spill.  Without
// a bound the d = 64 kernels took 260-320 registers, one wave per SIMD.
template <int DP>
constexpr int swa_bwd_occupancy() {
  return DP <= 32 ? 3 : DP <= 64 ? 2 : 1;
}

// ----------------------------------------------------------------------------
// backward, query side: delta (first pass over the window keys), dq (second
// pass), and this block's partial of dmeta
// ----------------------------------------------------------------------------
// RES: the window's key tiles (at most SWA_RES of them) stay in LDS, one slot
// each: pass 0 streams them in with one barrier per tile, pass 1 reads them
// back with no loads and no barriers.  Otherwise both passes stream the tiles
// through one k and one v buffer.

template <int DP, typename OutT, bool VEC, bool RES>
__global__ __launch_bounds__(256, (swa_bwd_occupancy<DP>())) void swa_bwd_dq_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ meta, int n_meta, const float* __restrict__ lse,
    const bf16* __restrict__ dy, OutT* __restrict__ dq, float* __restrict__ delta_out,
    float* __restrict__ dmeta_part, int BH, int L, int d, int W, float scale, int per, int nx,
    int KG) {
  using Cfg = SwaCfg<DP>;
  constexpr int P = Cfg::P;
  constexpr int NSLOT = RES ? SWA_RES : 1;
  extern __shared__ __align__(16) char smem[];
  // k tile of slot i at smem + i TILE_BYTES, v tile at smem + (NSLOT + i) TILE_BYTES
  auto kslot = [&](int i) { return reinterpret_cast<bf16*>(smem + i * Cfg::TILE_BYTES); };
  auto vslot = [&](int i) { return reinterpret_cast<bf16*>(smem + (NSLOT + i) * Cfg::TILE_BYTES); };
  float* red = reinterpret_cast<float*>(smem + 2 * NSLOT * Cfg::TILE_BYTES);   // [4][SWA_META_BLOCK]

  const int nqb = (L + SWA_ROWS - 1) / SWA_ROWS;
  const int lb = xcd_block(blockIdx.x, per, nx);
  if (lb >= BH * nqb) return;
  const int bh = lb / nqb, qb = lb % nqb, Q0 = qb * SWA_ROWS;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 31, h = lane >> 5;
  const int q0 = Q0 + wave * 32, qi = q0 + col;
  const size_t base = (size_t)bh * L * d;
  const size_t kvbase = (size_t)(bh / KG) * L * d;   // k, v: the kv head (KG query heads share one)
  const bool vec = VEC || (d & 7) == 0;

  bf16x8 qreg[DP / 16], dyreg[DP / 16];
  own_rows<DP>(q + base, qi, L, d, h, vec, qreg);
  own_rows<DP>(dy + base, qi, L, d, h, vec, dyreg);
  const float lse_i = qi < L ? lse[(size_t)bh * L + qi] : 0.f;

  const int klo = (max(0, Q0 - W + 1) / SWA_TILE) * SWA_TILE;
  const int khi = min(L, Q0 + SWA_ROWS);
  float delta = 0.f;
  f32x16 dqa[DP / 32];
#pragma unroll
  for (int t = 0; t < DP / 32; ++t) dqa[t] = zero16();

  // the work of one key tile (keys t0 .. t0+63 in k_l, v_l): pass 0 adds to
  // delta = sum_t p dp, pass 1 forms ds and adds ds k to dq
  auto tile = [&](int pass, const bf16* k_l, const bf16* v_l, int t0) __attribute__((always_inline)) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int k0 = t0 + 32 * half;
      if (!blocks_meet(q0, k0, L, W)) continue;
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int kb = 0; kb < DP / 16; ++kb) {
        s = mfma(row_operand(k_l, P, 32 * half + col, 16 * kb, h), qreg[kb], s);
        dp = mfma(row_operand(v_l, P, 32 * half + col, 16 * kb, h), dyreg[kb], dp);
      }
      if (pass == 0) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = in_window(qi, k0 + acc_row(r, h), W) ? fexp(s[r] * scale - lse_i) : 0.f;
          delta += p * dp[r];
        }
      } else {
        bf16x8 ds[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = in_window(qi, k0 + acc_row(r, h), W) ? fexp(s[r] * scale - lse_i) : 0.f;
          ds[r >> 3][r & 7] = to_bf16(p * (dp[r] - delta));
        }
#pragma unroll
        for (int t = 0; t < DP / 32; ++t)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
            dqa[t] = mfma(tr_operand(k_l, P, 32 * half + 16 * kb, t * 32, lane), ds[kb], dqa[t]);
      }
    }
  };

  uint4 rk[Cfg::NL], rv[Cfg::NL];
  if constexpr (RES) {
    const int nt = (khi - klo + SWA_TILE - 1) / SWA_TILE;   // <= SWA_RES (the launcher's test)
    swa_load<DP>(rk, k + kvbase, klo, L, d, vec);
    swa_load<DP>(rv, v + kvbase, klo, L, d, vec);
    swa_store<DP>(rk, kslot(0));
    swa_store<DP>(rv, vslot(0));
    __syncthreads();
    for (int i = 0; i < nt; ++i) {
      const int t0 = klo + i * SWA_TILE;
      const bool more = i + 1 < nt;
      if (more) {
        swa_load<DP>(rk, k + kvbase, t0 + SWA_TILE, L, d, vec);
        swa_load<DP>(rv, v + kvbase, t0 + SWA_TILE, L, d, vec);
      }
      tile(0, kslot(i), vslot(i), t0);
      if (more) {   // slot i + 1 is not read before this barrier
        swa_store<DP>(rk, kslot(i + 1));
        swa_store<DP>(rv, vslot(i + 1));
        __syncthreads();
      }
    }
    delta += xhalf(delta);
    for (int i = 0; i < nt; ++i) tile(1, kslot(i), vslot(i), klo + i * SWA_TILE);
  } else {
    // pass 0 accumulates delta = sum_t p dp; pass 1 forms ds and dq
    for (int pass = 0; pass < 2; ++pass) {
      swa_load<DP>(rk, k + kvbase, klo, L, d, vec);
      swa_load<DP>(rv, v + kvbase, klo, L, d, vec);
      __syncthreads();
      swa_store<DP>(rk, kslot(0));
      swa_store<DP>(rv, vslot(0));
      __syncthreads();
      for (int t0 = klo; t0 < khi; t0 += SWA_TILE) {
        const bool more = t0 + SWA_TILE < khi;
        if (more) {
          swa_load<DP>(rk, k + kvbase, t0 + SWA_TILE, L, d, vec);
          swa_load<DP>(rv, v + kvbase, t0 + SWA_TILE, L, d, vec);
        }
        tile(pass, kslot(0), vslot(0), t0);
        if (more) {
          __syncthreads();
          swa_store<DP>(rk, kslot(0));
          swa_store<DP>(rv, vslot(0));
          __syncthreads();
        }
      }
      if (pass == 0) delta += xhalf(delta);
    }
  }
#pragma unroll
  for (int t = 0; t < DP / 32; ++t) store_acc_row<OutT>(dq + base, qi, t * 32, L, d, vec, dqa[t], scale, h);
  if (qi < L && h == 0) delta_out[(size_t)bh * L + qi] = delta;
  // dmeta partial of this block: -sum_i e^{meta_j - lse_i} delta_i, sinks in
  // passes of SWA_META_BLOCK (one wave sum per sink, then the four waves')
  for (int j0 = 0; j0 < n_meta; j0 += SWA_META_BLOCK) {
    const int nj = min(SWA_META_BLOCK, n_meta - j0);
    for (int jj = 0; jj < nj; ++jj) {
      float c = (qi < L && h == 0) ? fexp(meta[j0 + jj] - lse_i) * delta : 0.f;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off);
      if (lane == 0) red[wave * SWA_META_BLOCK + jj] = c;
    }
    __syncthreads();
    if ((int)threadIdx.x < nj) {
      const int jj = threadIdx.x;
      const float c = red[jj] + red[SWA_META_BLOCK + jj] + red[2 * SWA_META_BLOCK + jj] +
                      red[3 * SWA_META_BLOCK + jj];
      dmeta_part[((size_t)bh * nqb + qb) * n_meta + j0 + jj] = -c;
    }
    __syncthreads();
  }
}

// dmeta[j] = sum over `rows` partial rows of part[row][j], by the first 256
// threads of a workgroup, in passes of up to 256 sinks: thread (group g, sink
// j) sums partial rows g, g + groups, ...; thread j then sums the groups, in a
// fixed order.  sh: 256 floats of LDS.
__device__ void dmeta_sum(const float* __restrict__ part, int rows, int n_meta,
                          float* __restrict__ dmeta, float* sh) {
  const int per = min(n_meta, 256), groups = 256 / per;
  for (int j0 = 0; j0 < n_meta; j0 += per) {
    const int nj = min(per, n_meta - j0);
    const int j = threadIdx.x % per, grp = threadIdx.x / per;
    float acc = 0.f;
    if (threadIdx.x < 256 && grp < groups && j < nj)
      for (int r = grp; r < rows; r += groups) acc += part[(size_t)r * n_meta + j0 + j];
    if (threadIdx.x < 256) sh[threadIdx.x] = acc;
    __syncthreads();
    if ((int)threadIdx.x < nj) {
      float t = 0.f;
      for (int g = 0; g < groups; ++g) t += sh[g * per + threadIdx.x];
      dmeta[j0 + threadIdx.x] = t;
    }
    __syncthreads();
  }
}

// ----------------------------------------------------------------------------
// backward, key side: dk and dv over the queries whose windows hold the keys
// ----------------------------------------------------------------------------
template <int DP, typename OutT, bool VEC>
__global__ __launch_bounds__(256, (swa_bwd_occupancy<DP>())) void swa_bwd_dkv_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ lse, const float* __restrict__ delta_in,
    const bf16* __restrict__ dy, OutT* __restrict__ dk, OutT* __restrict__ dv,
    const float* __restrict__ dmeta_part, float* __restrict__ dmeta, int n_meta, int BH, int L,
    int d, int W, float scale, int per, int nx, int KG) {
  using Cfg = SwaCfg<DP>;
  constexpr int P = Cfg::P;
  extern __shared__ __align__(16) char smem[];
  bf16* q_l = reinterpret_cast<bf16*>(smem);
  bf16* dy_l = reinterpret_cast<bf16*>(smem + Cfg::TILE_BYTES);
  float* lse_l = reinterpret_cast<float*>(smem + 2 * Cfg::TILE_BYTES);   // [64]
  float* del_l = lse_l + SWA_TILE;                                        // [64]

  const int nkb = (L + SWA_ROWS - 1) / SWA_ROWS;
  const int lb = xcd_block(blockIdx.x, per, nx);
  if (lb >= BH * nkb) return;
  // dmeta from the query-side blocks' partials (that launch has completed)
  if (lb == 0 && n_meta > 0) dmeta_sum(dmeta_part, BH * nkb, n_meta, dmeta, reinterpret_cast<float*>(smem));
  const int bh = lb / nkb, K0 = (lb % nkb) * SWA_ROWS;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const int k0 = K0 + wave * 32, ti = k0 + col;
  const size_t base = (size_t)bh * L * d, lbase = (size_t)bh * L;
  const size_t kvbase = (size_t)(bh / KG) * L * d;   // k, v: the kv head (KG query heads share one)
  const bool vec = VEC || (d & 7) == 0;

  bf16x8 kreg[DP / 16], vreg[DP / 16];
  own_rows<DP>(k + kvbase, ti, L, d, h, vec, kreg);
  own_rows<DP>(v + kvbase, ti, L, d, h, vec, vreg);
  f32x16 dka[DP / 32], dva[DP / 32];
#pragma unroll
  for (int t = 0; t < DP / 32; ++t) {
    dka[t] = zero16();
    dva[t] = zero16();
  }

  const int qlo = K0, qhi = min(L, K0 + SWA_ROWS - 1 + W);
  uint4 rq[Cfg::NL], rd[Cfg::NL];
  float rl = 0.f, rdl = 0.f;
  auto load_rows = [&](int r0) {
    swa_load<DP>(rq, q + base, r0, L, d, vec);
    swa_load<DP>(rd, dy + base, r0, L, d, vec);
    if (tid < SWA_TILE) {
      const bool ok = r0 + tid < L;
      rl = ok ? lse[lbase + r0 + tid] : 0.f;
      rdl = ok ? delta_in[lbase + r0 + tid] : 0.f;
    }
  };
  auto store_rows = [&]() {
    swa_store<DP>(rq, q_l);
    swa_store<DP>(rd, dy_l);
    if (tid < SWA_TILE) {
      lse_l[tid] = rl;
      del_l[tid] = rdl;
    }
  };
  load_rows(qlo);
  store_rows();
  __syncthreads();
  for (int t0 = qlo; t0 < qhi; t0 += SWA_TILE) {
    const bool more = t0 + SWA_TILE < qhi;
    if (more) load_rows(t0 + SWA_TILE);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const int qq0 = t0 + 32 * half;
      if (!blocks_meet(qq0, k0, L, W)) continue;
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int kb = 0; kb < DP / 16; ++kb) {
        s = mfma(row_operand(q_l, P, 32 * half + col, 16 * kb, h), kreg[kb], s);
        dp = mfma(row_operand(dy_l, P, 32 * half + col, 16 * kb, h), vreg[kb], dp);
      }
      // lane owns key ti; register r owns query qq0 + acc_row(r, h).  The
      // queries of registers 4 g .. 4 g + 3 are consecutive: their lse and
      // delta come in as 16-byte LDS reads, and the window is a select
      bf16x8 pb[2], dsb[2];
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int qr0 = 32 * half + 8 * g4 + 4 * h;
        const f32x4 ls = *reinterpret_cast<const f32x4*>(lse_l + qr0);
        const f32x4 dl = *reinterpret_cast<const f32x4*>(del_l + qr0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g4 + e;
          const float p = in_window(t0 + qr0 + e, ti, W) ? fexp(s[r] * scale - ls[e]) : 0.f;
          pb[r >> 3][r & 7] = to_bf16(p);
          dsb[r >> 3][r & 7] = to_bf16(p * (dp[r] - dl[e]));
        }
      }
#pragma unroll
      for (int t = 0; t < DP / 32; ++t)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          dva[t] = mfma(tr_operand(dy_l, P, 32 * half + 16 * kb, t * 32, lane), pb[kb], dva[t]);
          dka[t] = mfma(tr_operand(q_l, P, 32 * half + 16 * kb, t * 32, lane), dsb[kb], dka[t]);
        }
    }
    if (more) {
      __syncthreads();
      store_rows();
      __syncthreads();
    }
  }
#pragma unroll
  for (int t = 0; t < DP / 32; ++t) {
    store_acc_row<OutT>(dk + base, ti, t * 32, L, d, vec, dka[t], scale, h);
    store_acc_row<OutT>(dv + base, ti, t * 32, L, d, vec, dva[t], 1.f, h);
  }
}

// ----------------------------------------------------------------------------
// backward in one pass, for windows W <= 64 at d <= 64 (padded to 64)
//
// With W <= 64 the queries of 64-row block i see keys of blocks i - 1 and i
// only, and the keys of block j are seen by the queries of blocks j and j + 1.
// A workgroup of eight waves walks a segment of blocks b0 .. b1 - 1 of one
// (b, h); step i scores query block i against key blocks i - 1 and i once and
// uses the scores three times:
//   phase 1a  waves 0-5: pair (query half A, 32-key sub-block s), s = A .. A+2
//             of the four sub-blocks of blocks i - 1, i: S, dP = dy v^T, p and
//             the pair's part of delta = sum_t p dp (the fp32 form of the two
//             kernels above, no delta buffer);
//   phase 1b  delta = the three parts of the query half in key order;
//             ds = p (dp - delta); p and ds to LDS as bf16 [query][key] tiles;
//             the next block's rows (loaded a step ahead) to their LDS slots;
//   phase 2   waves 0-3: dq tile (A, t) = scale ds K over the three
//             sub-blocks: the query block is done, stored;
//             waves 4-7: key half kh of the block of parity par in {i-1, i}
//             accumulates dk += scale ds^T Q, dv += p^T dY; block i - 1 has
//             seen all its queries and is stored.
// The step past the segment (block b1, the next segment's first) runs for the
// dk, dv of block b1 - 1 only; the first step reads block b0 - 1's keys for
// the first queries' windows only.  Key tiles rotate through three LDS slots
// (blocks i - 1 and i read, i + 1 written), query and dy tiles through two.
// dmeta_j = -sum_i e^{meta_j - lse_i} delta_i = -e^{meta_j - m} T with
// m = max_j meta_j and T = sum_i e^{m - lse_i} delta_i (both factors at most 1,
// since lse_i >= m): a workgroup adds its queries' terms of T as it forms their
// deltas, and a second launch sums the workgroups' T in a fixed order.
// ----------------------------------------------------------------------------
constexpr int SWA_WALK_MAX_NB = 32;   // blocks per segment
constexpr int SWA_WALK_WAVES = 8;

struct SwaWalk {
  static constexpr int P = SwaCfg<64>::P;             // k, v, q, dy tiles [64][P]
  static constexpr int TB = SwaCfg<64>::TILE_BYTES;
  static constexpr int PP = lds_pitch(128);           // p, ds tiles [64 queries][PP]
  static constexpr int OFF_K = 0;                     // three k slots
  static constexpr int OFF_V = OFF_K + 3 * TB;        // three v slots
  static constexpr int OFF_Q = OFF_V + 3 * TB;        // two q buffers
  static constexpr int OFF_DY = OFF_Q + 2 * TB;       // two dy buffers
  static constexpr int OFF_P = OFF_DY + 2 * TB;
  static constexpr int OFF_DS = OFF_P + 64 * PP * 2;
  static constexpr int OFF_LSE = OFF_DS + 64 * PP * 2;            // [2][64] f32
  static constexpr int OFF_RED = OFF_LSE + 2 * 64 * 4;            // [6][32] f32
  static constexpr int LDS = OFF_RED + 6 * 32 * 4;
  static_assert(LDS <= 160 * 1024, "LDS budget");
  static_assert(SWA_TILE == 64 && SwaCfg<64>::NL * 256 == 64 * 8, "tile items");
};

// NTQ: the q and dy tiles load nontemporally (each is read by one walk),
// which leaves the caches to the k and v tiles that KG > 1 query heads share
// (config 5: 103.6 -> 98.2 us; at config 3, KG = 1, it read 21.6 -> 22.0 us)
template <typename OutT, bool VEC, bool NTQ = false>
__global__ __launch_bounds__(64 * SWA_WALK_WAVES, 1) void swa_bwd_walk_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ meta, int n_meta, const float* __restrict__ lse,
    const bf16* __restrict__ dy, OutT* __restrict__ dq, OutT* __restrict__ dk,
    OutT* __restrict__ dv, float* __restrict__ dmeta_part, int BH, int L, int d, int W,
    float scale, int NB, int nseg, int per, int nx, int KG) {
  using C = SwaWalk;
  constexpr int P = C::P, PP = C::PP, NT = 64 * SWA_WALK_WAVES;
  extern __shared__ __align__(16) char smem[];
  auto kslot = [&](int j) { return reinterpret_cast<bf16*>(smem + C::OFF_K + ((j + 3) % 3) * C::TB); };
  auto vslot = [&](int j) { return reinterpret_cast<bf16*>(smem + C::OFF_V + ((j + 3) % 3) * C::TB); };
  auto qbuf = [&](int j) { return reinterpret_cast<bf16*>(smem + C::OFF_Q + (j & 1) * C::TB); };
  auto dybuf = [&](int j) { return reinterpret_cast<bf16*>(smem + C::OFF_DY + (j & 1) * C::TB); };
  auto lsebuf = [&](int j) { return reinterpret_cast<float*>(smem + C::OFF_LSE) + (j & 1) * 64; };
  bf16* p_l = reinterpret_cast<bf16*>(smem + C::OFF_P);
  bf16* ds_l = reinterpret_cast<bf16*>(smem + C::OFF_DS);
  float* red = reinterpret_cast<float*>(smem + C::OFF_RED);

  const int lb = xcd_block(blockIdx.x, per, nx);
  if (lb >= BH * nseg) return;
  const int bh = lb / nseg, seg = lb % nseg;
  const int nblk = (L + SWA_TILE - 1) / SWA_TILE;
  const int b0 = seg * NB, b1 = min(nblk, b0 + NB);
  const int iend = min(b1, nblk - 1);   // the step past the segment, when there is a block
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, col = lane & 31, h = lane >> 5;
  const size_t base = (size_t)bh * L * d, kvbase = (size_t)(bh / KG) * L * d;
  const bf16 *qb = q + base, *dyb = dy + base, *kb = k + kvbase, *vb = v + kvbase;
  const float* lseb = lse + (size_t)bh * L;
  const bool vec = VEC || (d & 7) == 0;

  // one 16-byte item per thread of a 64-row tile (row tid / 8, columns
  // 8 (tid % 8)); rows outside [0, L) read zero
  auto load_tile = [&](uint4& r, const bf16* src, int r0) {
    uint4 t[1];
    load_items<64, NT, 1, NT>(t, src, r0, L, d, vec);
    r = t[0];
  };
  auto load_qd = [&](uint4& r, const bf16* src, int r0) {   // a q or dy tile
    uint4 t[1];
    load_items<64, NT, 1, NT, NTQ ? LOAD_NT : 0>(t, src, r0, L, d, vec);
    r = t[0];
  };
  auto store_tile = [&](const uint4& r, bf16* tile) {
    *reinterpret_cast<uint4*>(tile + (tid >> 3) * P + (tid & 7) * 8) = r;
  };
  // lse of a block's 64 rows: every thread loads row tid % 64 and writes it to
  // LDS (eight equal writes per row), so neither the load nor the write sits
  // under a branch: a branch there leaves the compiler unsure whether the load
  // is still in flight, and its wait before the next one also drains the
  // output stores issued in between
  const rsrc_t lse_r = make_rsrc(lseb, (size_t)L * 4);
  auto load_lse = [&](int r0) {
    const int r = r0 + (tid & 63);
    return bload_f32(lse_r, r < L ? (uint32_t)r * 4u : OOB);
  };

  // the first step's rows: key block b0 - 1 (zero rows before the sequence),
  // block b0; the next block's rows stay in registers until step b0 stores them
  uint4 pk, pv, pq, pd;
  float pl;
  {
    uint4 k0r, v0r;
    load_tile(k0r, kb, SWA_TILE * (b0 - 1));
    load_tile(v0r, vb, SWA_TILE * (b0 - 1));
    load_tile(pk, kb, SWA_TILE * b0);
    load_tile(pv, vb, SWA_TILE * b0);
    load_qd(pq, qb, SWA_TILE * b0);
    load_qd(pd, dyb, SWA_TILE * b0);
    pl = load_lse(SWA_TILE * b0);
    store_tile(k0r, kslot(b0 - 1));
    store_tile(v0r, vslot(b0 - 1));
    store_tile(pk, kslot(b0));
    store_tile(pv, vslot(b0));
    store_tile(pq, qbuf(b0));
    store_tile(pd, dybuf(b0));
    lsebuf(b0)[tid & 63] = pl;
    if (b0 + 1 <= iend) {
      load_tile(pk, kb, SWA_TILE * (b0 + 1));
      load_tile(pv, vb, SWA_TILE * (b0 + 1));
      load_qd(pq, qb, SWA_TILE * (b0 + 1));
      load_qd(pd, dyb, SWA_TILE * (b0 + 1));
      pl = load_lse(SWA_TILE * (b0 + 1));
    }
  }
  __syncthreads();

  // phase-1 pair of this wave (waves 0-5) and phase-2 role
  const int pA = wave / 3, psub = pA + wave % 3;
  f32x16 acc[4];   // waves 0-3: acc[0] = dq tile; waves 4-7: dk tiles 0-1, dv tiles 0-1
#pragma unroll
  for (int t = 0; t < 4; ++t) acc[t] = zero16();
  // this lane's terms of T (waves 0 and 3, lane half 0: one query row each)
  float mmax = -1e30f;
  for (int j = 0; j < n_meta; ++j) mmax = fmaxf(mmax, meta[j]);
  float tpart = 0.f;
  int out_row = -1;   // row of this lane's finished tile (dq: query, dk/dv: key); -1: none
  auto flush = [&]() {
    if (wave < 4) {
      if (out_row >= 0)
        store_acc_row<OutT>(dq + base, out_row, 32 * (wave & 1), L, d, vec, acc[0], scale, h);
      acc[0] = zero16();
    } else if (out_row >= 0) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        store_acc_row<OutT>(dk + base, out_row, 32 * t, L, d, vec, acc[t], scale, h);
        store_acc_row<OutT>(dv + base, out_row, 32 * t, L, d, vec, acc[2 + t], 1.f, h);
        acc[t] = zero16();
        acc[2 + t] = zero16();
      }
    }
    out_row = -1;
  };

  for (int i = b0; i <= iend; ++i) {
    const bool own_q = i < b1;
    // ---- 1a. scores of the wave's pair; its part of delta -------------------
    const int key0 = SWA_TILE * (i - 1) + 32 * psub, q0 = SWA_TILE * i + 32 * pA, qi = q0 + col;
    const bool pair = wave < 6 && key0 >= 0 && blocks_meet(q0, key0, L, W);
    f32x16 pr = zero16(), dpr = zero16();
    float dpart = 0.f;
    const float lq = wave < 6 ? lsebuf(i)[32 * pA + col] : 0.f;
    if (pair) {
      const bf16* kt = psub < 2 ? kslot(i - 1) : kslot(i);
      const bf16* vt = psub < 2 ? vslot(i - 1) : vslot(i);
      const bf16* qt = qbuf(i);
      const bf16* dyt = dybuf(i);
      f32x16 s = zero16();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        s = mfma(row_operand(kt, P, 32 * (psub & 1) + col, 16 * kk, h),
                 row_operand(qt, P, 32 * pA + col, 16 * kk, h), s);
        dpr = mfma(row_operand(vt, P, 32 * (psub & 1) + col, 16 * kk, h),
                   row_operand(dyt, P, 32 * pA + col, 16 * kk, h), dpr);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool ok = qi < L && in_window(qi, key0 + acc_row(r, h), W);
        pr[r] = ok ? fexp(s[r] * scale - lq) : 0.f;
        dpart += pr[r] * dpr[r];
      }
      dpart += xhalf(dpart);
    }
    if (wave < 6 && h == 0) red[wave * 32 + col] = dpart;   // zero for an empty pair
    __syncthreads();

    // ---- 1b. delta; p and ds to LDS; the next block's rows to their slots ----
    if (wave < 6) {
      const float* rr = red + 3 * pA * 32 + col;
      const float del = rr[0] + rr[32] + rr[64];
      if (pair) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          bf16x4 p4, d4;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g + e;
            p4[e] = to_bf16(pr[r]);
            d4[e] = to_bf16(pr[r] * (dpr[r] - del));
          }
          const int at = (32 * pA + col) * PP + 32 * psub + 8 * g + 4 * h;
          *reinterpret_cast<bf16x4*>(p_l + at) = p4;
          *reinterpret_cast<bf16x4*>(ds_l + at) = d4;
        }
      }
      if (wave % 3 == 0 && h == 0 && own_q && qi < L) tpart += fexp(mmax - lq) * del;
    }
    if (i + 1 <= iend) {   // slots of blocks i - 2 and i - 1: their last readers passed the barrier
      store_tile(pk, kslot(i + 1));
      store_tile(pv, vslot(i + 1));
      store_tile(pq, qbuf(i + 1));
      store_tile(pd, dybuf(i + 1));
      lsebuf(i + 1)[tid & 63] = pl;
    }
    if (i + 1 <= iend) {
      if (i + 2 <= iend) {
        load_tile(pk, kb, SWA_TILE * (i + 2));
        load_tile(pv, vb, SWA_TILE * (i + 2));
        load_qd(pq, qb, SWA_TILE * (i + 2));
        load_qd(pd, dyb, SWA_TILE * (i + 2));
        pl = load_lse(SWA_TILE * (i + 2));
      }
    }
    __syncthreads();

    // ---- 2. dq of query block i; dk, dv of key blocks i - 1 and i ------------
    if (wave < 4) {
      const int A = wave >> 1, t = wave & 1, qa = SWA_TILE * i + 32 * A;
      if (own_q) {
#pragma unroll
        for (int s3 = 0; s3 < 3; ++s3) {
          const int sub = A + s3, kk0 = SWA_TILE * (i - 1) + 32 * sub;
          if (kk0 < 0 || !blocks_meet(qa, kk0, L, W)) continue;
          const bf16* kt = sub < 2 ? kslot(i - 1) : kslot(i);
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
            acc[0] = mfma(tr_operand_c(kt, P, 32 * (sub & 1) + 16 * kk, 32 * t, lane),
                          row_operand(ds_l, PP, 32 * A + col, 32 * sub + 16 * kk, h), acc[0]);
        }
        out_row = qa + col;
        flush();
      }
    } else {
      const int par = (wave - 4) >> 1, kh = (wave - 4) & 1;
      const int j = (i & 1) == par ? i : i - 1;
      if (j >= b0 && j < b1) {   // a block of this segment
        const int sub = (j == i ? 2 : 0) + kh, kk0 = SWA_TILE * j + 32 * kh;
#pragma unroll
        for (int A = 0; A < 2; ++A) {
          if (sub < A || sub > A + 2 || !blocks_meet(SWA_TILE * i + 32 * A, kk0, L, W)) continue;
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) {
            const bf16x8 bds = tr_operand_c(ds_l, PP, 32 * A + 16 * kk, 32 * sub, lane);
            const bf16x8 bp = tr_operand_c(p_l, PP, 32 * A + 16 * kk, 32 * sub, lane);
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              acc[t] = mfma(tr_operand_c(qbuf(i), P, 32 * A + 16 * kk, 32 * t, lane), bds, acc[t]);
              acc[2 + t] = mfma(tr_operand_c(dybuf(i), P, 32 * A + 16 * kk, 32 * t, lane), bp,
                                acc[2 + t]);
            }
          }
        }
        if (j == i - 1 || j == nblk - 1) out_row = kk0 + col;   // every query of block j is in
        flush();
      }
    }
  }
  flush();

  // ---- this workgroup's T --------------------------------------------------
  if (n_meta > 0) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) tpart += __shfl_xor(tpart, off);
    __syncthreads();   // every reader of red is past it
    if (lane == 0 && wave % 3 == 0 && wave < 6) red[wave / 3] = tpart;
    __syncthreads();
    if (tid == 0) dmeta_part[lb] = red[0] + red[1];
  }
}

// dmeta_j = -e^{meta_j - m} sum_w T_w, the workgroups' T summed in a fixed
// order by one wave (strided lane sums, then a butterfly).  The lane's sink
// logit and its first 16 partials are loaded together, before any is used
// (buffer loads, zero past the end), so the kernel waits one memory round
// trip for up to 1024 partials, not one per 64; each lane still adds its
// partials in row order, from zero.
__global__ __launch_bounds__(64) void swa_dmeta_reduce_kernel(const float* __restrict__ part,
                                                              int rows, const float* __restrict__ meta,
                                                              int n_meta, float* __restrict__ dmeta) {
  const int lane = threadIdx.x;
  constexpr int U = 16;
  const rsrc_t src = make_rsrc(part, (size_t)rows * 4);
  const float m0 = lane < n_meta ? meta[lane] : -1e30f;
  float t = 0.f;
  for (int r0 = 0; r0 < rows; r0 += 64 * U) {
    float x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r = r0 + 64 * u + lane;
      x[u] = bload_f32(src, r < rows ? (uint32_t)r * 4u : OOB);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) t += x[u];
  }
  float mmax = fmaxf(-1e30f, m0);
  for (int j = lane + 64; j < n_meta; j += 64) mmax = fmaxf(mmax, meta[j]);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    t += __shfl_xor(t, off);
    mmax = fmaxf(mmax, __shfl_xor(mmax, off));
  }
  if (lane < n_meta) dmeta[lane] = -fexp(m0 - mmax) * t;
  for (int j = lane + 64; j < n_meta; j += 64) dmeta[j] = -fexp(meta[j] - mmax) * t;
}

// ----------------------------------------------------------------------------
// host launchers
// ----------------------------------------------------------------------------
int swa_padded_dim(int d) {
  if (d <= 32) return 32;
  if (d <= 64) return 64;
  if (d <= 128) return 128;
  if (d <= 256) return 256;
  return -1;
}

// blocks per (b, h) and the XCD-spread grid for BH * nblk logical blocks
static void swa_grid(int BH, int L, int* per, int* grid, int* nx) {
  const int nblk = (L + SWA_ROWS - 1) / SWA_ROWS;
  *nx = device_geom().xcds;
  *grid = xcd_grid(BH * nblk, *nx);
  *per = *grid / *nx;
}

int swa_row_blocks(int L) { return (L + SWA_ROWS - 1) / SWA_ROWS; }

template <int DP, bool VEC, bool RES>
static hipError_t launch_swa_fwd_r(const void* q, const void* k, const void* v, const float* meta,
                                   int n_meta, void* y, float* lse, int BH, int L, int d, int W,
                                   float scale, int KG, hipStream_t st) {
  const size_t lds = 2 * (RES ? SWA_RES : 1) * SwaCfg<DP>::TILE_BYTES;
  hipError_t e = ensure_lds<swa_fwd_kernel<DP, VEC, RES>>((int)lds);
  if (e != hipSuccess) return e;
  int per, grid, nx;
  swa_grid(BH, L, &per, &grid, &nx);
  hipLaunchKernelGGL((swa_fwd_kernel<DP, VEC, RES>), dim3(grid), dim3(256), lds, st,
                     (const bf16*)q, (const bf16*)k, (const bf16*)v, meta, n_meta, (bf16*)y, lse,
                     BH, L, d, W, scale, per, nx, KG);
  return hipGetLastError();
}

template <int DP, bool VEC>
static hipError_t launch_swa_fwd_t(const void* q, const void* k, const void* v, const float* meta,
                                   int n_meta, void* y, float* lse, int BH, int L, int d, int W,
                                   float scale, int KG, hipStream_t st) {
  // resident tiles at d <= 64 when a block's keys span at most SWA_RES tiles
  // (SWA_ROWS + W + 62 <= SWA_RES * SWA_TILE, as the dq kernel's) and the
  // grid is at most two workgroups per CU (the slots allow two per CU)
  if constexpr (DP <= 64) {
    if (SWA_ROWS + W + 62 <= SWA_RES * SWA_TILE &&
        BH * swa_row_blocks(L) <= 2 * device_geom().cus)
      return launch_swa_fwd_r<DP, VEC, true>(q, k, v, meta, n_meta, y, lse, BH, L, d, W, scale,
                                             KG, st);
  }
  return launch_swa_fwd_r<DP, VEC, false>(q, k, v, meta, n_meta, y, lse, BH, L, d, W, scale, KG,
                                          st);
}

// Blocks per segment of the one-pass backward: enough segments for one
// workgroup per CU where the rows allow, at least two blocks per segment when
// there are two (so there are no more segments than the two-kernel form's
// 128-row blocks, whose dmeta partial rows the workspace holds).
static int swa_walk_blocks(int BH, int L) {
  const int nblk = (L + SWA_TILE - 1) / SWA_TILE;
  const int cus = device_geom().cus;
  int nb = (BH * nblk + cus - 1) / cus;
  nb = max(nb, nblk >= 2 ? 2 : 1);
  return min(min(nb, SWA_WALK_MAX_NB), nblk);
}

template <typename OutT, bool VEC>
static hipError_t launch_swa_bwd_walk(const void* q, const void* k, const void* v,
                                      const float* meta, int n_meta, const float* lse,
                                      const void* dy, void* dq, void* dk, void* dv,
                                      float* dmeta_part, float* dmeta, int BH, int L, int d, int W,
                                      float scale, int KG, hipStream_t st) {
  const int nblk = (L + SWA_TILE - 1) / SWA_TILE;
  const int NB = swa_walk_blocks(BH, L), nseg = (nblk + NB - 1) / NB;
  const int nx = device_geom().xcds, grid = xcd_grid(BH * nseg, nx), per = grid / nx;
  auto launch = [&](auto tag) {
    constexpr auto kern = decltype(tag)::value;
    if (hipError_t e2 = ensure_lds<kern>(SwaWalk::LDS); e2 != hipSuccess) return e2;
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * SWA_WALK_WAVES), SwaWalk::LDS, st,
                       (const bf16*)q, (const bf16*)k, (const bf16*)v, meta, n_meta, lse,
                       (const bf16*)dy, (OutT*)dq, (OutT*)dk, (OutT*)dv, dmeta_part, BH, L, d, W,
                       scale, NB, nseg, per, nx, KG);
    return hipGetLastError();
  };
  hipError_t e = KG > 1 ? launch(KernTag<swa_bwd_walk_kernel<OutT, VEC, true>>{})
                        : launch(KernTag<swa_bwd_walk_kernel<OutT, VEC>>{});
  if (e != hipSuccess || n_meta == 0) return e;
  hipLaunchKernelGGL(swa_dmeta_reduce_kernel, dim3(1), dim3(64), 0, st,
                     (const float*)dmeta_part, BH * nseg, meta, n_meta, dmeta);
  return hipGetLastError();
}

template <int DP, typename OutT, bool VEC>
static hipError_t launch_swa_bwd_t(const void* q, const void* k, const void* v, const float* meta,
                                   int n_meta, const float* lse, const void* dy, void* dq,
                                   void* dk, void* dv, float* delta, float* dmeta_part,
                                   float* dmeta, int BH, int L, int d, int W, float scale, int KG,
                                   hipStream_t st) {
  // W <= 64 at d <= 64: the one-pass walk (no delta buffer)
  if constexpr (DP == 64) {
    if (W <= SWA_TILE)
      return launch_swa_bwd_walk<OutT, VEC>(q, k, v, meta, n_meta, lse, dy, dq, dk, dv, dmeta_part,
                                            dmeta, BH, L, d, W, scale, KG, st);
  }
  int per, grid, nx;
  swa_grid(BH, L, &per, &grid, &nx);
  // the window's key tiles fit the LDS slots of the resident form when a
  // block's keys span at most SWA_RES tiles: klo >= Q0 - W - 62, khi <= Q0 +
  // SWA_ROWS, so SWA_ROWS + W + 62 <= SWA_RES * SWA_TILE; and at d <= 64,
  // where the slots leave the kernel's workgroups per CU in place
  const bool res = DP <= 64 && SWA_ROWS + W + 62 <= SWA_RES * SWA_TILE;
  hipError_t e;
  const size_t lds_q = 2 * (res ? SWA_RES : 1) * SwaCfg<DP>::TILE_BYTES +
                       4 * SWA_META_BLOCK * sizeof(float);
  if (res) {
    if ((e = ensure_lds<swa_bwd_dq_kernel<DP, OutT, VEC, true>>((int)lds_q)) != hipSuccess) return e;
    hipLaunchKernelGGL((swa_bwd_dq_kernel<DP, OutT, VEC, true>), dim3(grid), dim3(256), lds_q, st,
                       (const bf16*)q, (const bf16*)k, (const bf16*)v, meta, n_meta, lse,
                       (const bf16*)dy, (OutT*)dq, delta, dmeta_part, BH, L, d, W, scale, per, nx,
                       KG);
  } else {
    if ((e = ensure_lds<swa_bwd_dq_kernel<DP, OutT, VEC, false>>((int)lds_q)) != hipSuccess) return e;
    hipLaunchKernelGGL((swa_bwd_dq_kernel<DP, OutT, VEC, false>), dim3(grid), dim3(256), lds_q, st,
                       (const bf16*)q, (const bf16*)k, (const bf16*)v, meta, n_meta, lse,
                       (const bf16*)dy, (OutT*)dq, delta, dmeta_part, BH, L, d, W, scale, per, nx,
                       KG);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const size_t lds_k = 2 * SwaCfg<DP>::TILE_BYTES + 2 * SWA_TILE * sizeof(float);
  auto kk = swa_bwd_dkv_kernel<DP, OutT, VEC>;
  if ((e = ensure_lds<swa_bwd_dkv_kernel<DP, OutT, VEC>>((int)lds_k)) != hipSuccess) return e;
  hipLaunchKernelGGL(kk, dim3(grid), dim3(256), lds_k, st, (const bf16*)q, (const bf16*)k,
                     (const bf16*)v, lse, (const float*)delta, (const bf16*)dy, (OutT*)dk,
                     (OutT*)dv, (const float*)dmeta_part, dmeta, n_meta, BH, L, d, W, scale, per,
                     nx, KG);
  return hipGetLastError();
}

hipError_t launch_swa_fwd(const void* q, const void* k, const void* v, const float* meta,
                          int n_meta, void* y, float* lse, int BH, int L, int d, int W,
                          float scale, int KG, hipStream_t st) {
  const bool vec = d % 8 == 0;
#define LZ_SWA_FWD(DPV)                                                                         \
  return vec ? launch_swa_fwd_t<DPV, true>(q, k, v, meta, n_meta, y, lse, BH, L, d, W, scale,   \
                                           KG, st)                                              \
             : launch_swa_fwd_t<DPV, false>(q, k, v, meta, n_meta, y, lse, BH, L, d, W, scale,  \
                                            KG, st)
  switch (swa_padded_dim(d)) {
    case 32: LZ_SWA_FWD(32);
    case 64: LZ_SWA_FWD(64);
    case 128: LZ_SWA_FWD(128);
    case 256: LZ_SWA_FWD(256);
    default: return hipErrorInvalidValue;
  }
#undef LZ_SWA_FWD
}

hipError_t launch_swa_bwd(const void* q, const void* k, const void* v, const float* meta,
                          int n_meta, const float* lse, const void* dy, void* dq, void* dk,
                          void* dv, bool grad_bf16, float* delta, float* dmeta_part,
                          float* dmeta, int BH, int L, int d, int W, float scale, int KG,
                          hipStream_t st) {
  const bool vec = d % 8 == 0;
#define LZ_SWA_BWD_V(DPV, OUT, V)                                                               \
  launch_swa_bwd_t<DPV, OUT, V>(q, k, v, meta, n_meta, lse, dy, dq, dk, dv, delta, dmeta_part, \
                                dmeta, BH, L, d, W, scale, KG, st)
#define LZ_SWA_BWD(DPV)                                                                         \
  return grad_bf16 ? (vec ? LZ_SWA_BWD_V(DPV, bf16, true) : LZ_SWA_BWD_V(DPV, bf16, false))     \
                   : (vec ? LZ_SWA_BWD_V(DPV, float, true) : LZ_SWA_BWD_V(DPV, float, false))
  switch (swa_padded_dim(d)) {
    case 32: LZ_SWA_BWD(32);
    case 64: LZ_SWA_BWD(64);
    case 128: LZ_SWA_BWD(128);
    case 256: LZ_SWA_BWD(256);
    default: return hipErrorInvalidValue;
  }
#undef LZ_SWA_BWD
#undef LZ_SWA_BWD_V
}

// ----------------------------------------------------------------------------
// decode step: one new query per (b, h) against a ring-buffered window cache
//   keys/values of absolute positions pos - n + 1 .. pos, n = min(pos + 1, W),
//   position p in slot p % W of k_cache, v_cache [B*Hkv, W, d] (the caller
//   has written position pos there);
//   y = sum_p e^{s_p - m} v_p / (sum_j e^{meta_j - m} + sum_p e^{s_p - m}),
//   s_p = scale q . k_p, m = max(max_p s_p, max_j meta_j) -- the forward's
//   row at position pos (src/kernels/swa.py:19-59), with e^{s_p - m} rounded to
//   bf16 before it weights v, as the forward's P is.
// One workgroup per (b, h): thread t scores keys t, t + 256, ... (16-byte
// loads of its key rows when d % 8 == 0 and the cache is 16-byte aligned); the
// block takes the max and the sum; then thread (g, c) sums column c over keys
// g, g + NG, ... (NG = 256 / d groups, v rows read coalesced) and the groups'
// partial sums meet in LDS.
// ----------------------------------------------------------------------------
constexpr int SWA_DEC_MAX_W = 8192;

__device__ __forceinline__ float decode_max256(float* sh, float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x = fmaxf(x, __shfl_xor(x, off));
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = x;
  __syncthreads();
  x = fmaxf(fmaxf(sh[0], sh[1]), fmaxf(sh[2], sh[3]));
  __syncthreads();
  return x;
}

__device__ __forceinline__ float decode_sum256(float* sh, float x) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) x += __shfl_xor(x, off);
  if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = x;
  __syncthreads();
  x = (sh[0] + sh[1]) + (sh[2] + sh[3]);
  __syncthreads();
  return x;
}

__global__ __launch_bounds__(256) void swa_decode_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ kc, const bf16* __restrict__ vc,
    const float* __restrict__ meta, int n_meta, bf16* __restrict__ y, int W, int d, int pos,
    float scale, int KG) {
  extern __shared__ __align__(16) char smem[];
  float* w = reinterpret_cast<float*>(smem);        // [W] bf16-rounded weights
  float* qs = w + W;                                // [d] query
  float* part = qs + ((d + 3) & ~3);                // [256] column partial sums
  float* sh = part + 256;                           // [4] block reductions
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int n = min(pos + 1, W);
  const bf16* kb = kc + (size_t)(bh / KG) * W * d;
  const bf16* vb = vc + (size_t)(bh / KG) * W * d;
  const bool vec = (d & 7) == 0 && (reinterpret_cast<uintptr_t>(kb) & 15) == 0;
  for (int c = tid; c < d; c += 256) qs[c] = to_f32(q[(size_t)bh * d + c]);
  __syncthreads();
  float mx = -1e30f;
  for (int j = 0; j < n_meta; ++j) mx = fmaxf(mx, meta[j]);
  // scores, key i = tid, tid + 256, ... (position pos - n + 1 + i)
  for (int i = tid; i < n; i += 256) {
    const bf16* kr = kb + (size_t)((pos - n + 1 + i) % W) * d;
    float s = 0.f;
    if (vec) {
      for (int c = 0; c < d; c += 8) {
        const bf16x8 k8 = *reinterpret_cast<const bf16x8*>(kr + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) s += qs[c + e] * to_f32(k8[e]);
      }
    } else {
      for (int c = 0; c < d; ++c) s += qs[c] * to_f32(kr[c]);
    }
    s *= scale;
    w[i] = s;
    mx = fmaxf(mx, s);
  }
  const float m = decode_max256(sh, mx);
  float l = 0.f;
  for (int i = tid; i < n; i += 256) {
    const float e = fexp(w[i] - m);
    l += e;
    w[i] = to_f32(to_bf16(e));
  }
  l = decode_sum256(sh, l);   // also orders the weight writes before the reads below
  float ls = 0.f;
  for (int j = 0; j < n_meta; ++j) ls += fexp(meta[j] - m);
  const float inv = 1.f / (ls + l);
  const int NG = 256 / d, g = tid / d, c = tid - g * d;   // d <= 256: NG >= 1
  float acc = 0.f;
  if (g < NG) {
#pragma unroll 4
    for (int i = g; i < n; i += NG)
      acc += w[i] * to_f32(vb[(size_t)((pos - n + 1 + i) % W) * d + c]);
  }
  part[tid] = acc;
  __syncthreads();
  if (tid < d) {
    float t = part[tid];
    for (int j = 1; j < NG; ++j) t += part[j * d + tid];
    y[(size_t)bh * d + tid] = to_bf16(t * inv);
  }
}

size_t swa_decode_lds(int W, int d) {
  return ((size_t)W + ((d + 3) & ~3) + 256 + 4) * sizeof(float);
}

hipError_t launch_swa_decode(const void* q, const void* k_cache, const void* v_cache,
                             const float* meta, int n_meta, void* y, int BH, int W, int d,
                             int pos, float scale, int KG, hipStream_t st) {
  const size_t lds = swa_decode_lds(W, d);
  hipError_t e = ensure_lds<swa_decode_kernel>((int)swa_decode_lds(SWA_DEC_MAX_W, 256));
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(swa_decode_kernel, dim3(BH), dim3(256), lds, st, (const bf16*)q,
                     (const bf16*)k_cache, (const bf16*)v_cache, meta, n_meta, (bf16*)y, W, d,
                     pos, scale, KG);
  return hipGetLastError();
}

}  // namespace lz
