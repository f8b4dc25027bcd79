// Sliding-window softmax attention with learned sink logits, forward and
// backward, for gfx950.
//
// Math (reference: src/lizard_attention.py:34-44 dense form; operator API
// src/kernels/swa.py:136-183):
//   s_it = q_i . k_t / sqrt(d) for keys i-W < t <= i (t < L)
//   y_i  = sum_t e^{s_it} v_t / (sum_j e^{meta_j} + sum_t e^{s_it})
//   lse_i = log(sum_j e^{meta_j} + sum_t e^{s_it})
// Backward with delta_i = dy_i . y_i (src/kernels/swa.py:164).  The reference
// takes y from the bf16 output; here the forward also keeps y in fp32 (y32)
// when a backward will follow, and delta uses it: with bf16 y the sink
// gradient alone loses ~1 % to the rounding (it is a long signed sum of delta).
//   p_it = e^{s_it - lse_i},  ds_it = p_it (dy_i . v_t - delta_i)
//   dq_i = scale sum_t ds_it k_t,  dk_t = scale sum_i ds_it q_i,
//   dv_t = sum_i p_it dy_i,  dmeta_j = -sum_i e^{meta_j - lse_i} delta_i
//
// Layout: q, k, v, y, dy are [BH, L, d] bf16 row-major; y32 is [BH, L, d]
// fp32; lse is [BH, L] fp32.
// A workgroup is 4 waves; each wave owns a 32-row tile (queries in the
// forward and dq role, keys in the dk/dv role) and keeps its own rows in
// registers as MFMA operands.  The other side of each product is staged per
// 32-row tile in LDS, both natural ([row][d], for contractions over d) and
// transposed ([d][row], for contractions over rows).  Scores are computed
// transposed (keys x queries in the forward) so that each lane owns one query
// and the softmax statistics are per-lane scalars; P then feeds P*V straight
// from the accumulator registers (see common.hpp).
#include "common.hpp"

namespace lz {

constexpr int SWA_MAX_META = 64;

template <int DP>
struct SwaTiles {
  static constexpr int NPITCH = DP + 8;   // natural tile [32][NPITCH]
  static constexpr int TPITCH = 32 + 8;   // transposed tile [DP][TPITCH]
  static constexpr int NAT_ELEMS = 32 * NPITCH;
  static constexpr int TR_ELEMS = DP * TPITCH;
};

// Cooperatively stage rows [r0, r0+32) of a [nrows x ncols] matrix into a
// natural tile (slot order along d) and/or a transposed tile (slot order
// along rows).  256 threads.
template <int DP, bool NAT, bool TR>
__device__ __forceinline__ void stage_rows(const bf16* __restrict__ src, int r0, int nrows,
                                           int ncols, bf16* nat, bf16* tr) {
  using T = SwaTiles<DP>;
  constexpr int C4 = DP / 4;
  for (int idx = threadIdx.x; idx < 32 * C4; idx += 256) {
    const int r = idx / C4, c = (idx % C4) * 4;
    const bf16x4 x = load4(src, r0 + r, c, nrows, ncols);
    if constexpr (NAT) *reinterpret_cast<bf16x4*>(nat + r * T::NPITCH + pidx(c)) = x;
    if constexpr (TR) {
#pragma unroll
      for (int e = 0; e < 4; ++e) tr[(c + e) * T::TPITCH + pidx(r)] = x[e];
    }
  }
}

// Operand registers for a 32-row tile held by the wave: lane (row r0+l%32,
// half h) gets elements k = 16*kb + slot order, zero outside the matrix.
template <int DP>
__device__ __forceinline__ void load_rows_operand(const bf16* __restrict__ src, int row,
                                                  int nrows, int ncols, int h,
                                                  bf16x8 (&reg)[DP / 16]) {
#pragma unroll
  for (int kb = 0; kb < DP / 16; ++kb) {
    const bf16x4 lo = load4(src, row, 16 * kb + 4 * h, nrows, ncols);
    const bf16x4 hi = load4(src, row, 16 * kb + 8 + 4 * h, nrows, ncols);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      reg[kb][e] = lo[e];
      reg[kb][4 + e] = hi[e];
    }
  }
}

__device__ __forceinline__ bool in_window(int i, int t, int L, int W) {
  return t <= i && i - t < W && t < L && i < L;
}

// ----------------------------------------------------------------------------
// forward: grid (ceil(L/128), BH), 256 threads
// ----------------------------------------------------------------------------
template <int DP>
__global__ __launch_bounds__(256) void swa_fwd_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ meta, int n_meta, bf16* __restrict__ y, float* __restrict__ y32,
    float* __restrict__ lse, int L, int d, int W, float scale) {
  using T = SwaTiles<DP>;
  extern __shared__ __align__(16) char smem[];
  bf16* kn = reinterpret_cast<bf16*>(smem);
  bf16* vt = kn + T::NAT_ELEMS;

  const int bh = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 31, h = lane >> 5;
  const int Q0 = blockIdx.x * 128;
  const int q0 = Q0 + wave * 32;
  const size_t base = (size_t)bh * L * d;
  const int qi = q0 + col;

  bf16x8 qreg[DP / 16];
  load_rows_operand<DP>(q + base, qi, L, d, h, qreg);

  // running max and sum start from the sinks (src/kernels/swa.py:34-38)
  float m_i = -1e30f;
  for (int j = 0; j < n_meta; ++j) m_i = fmaxf(m_i, meta[j]);
  float l_i = 0.f;
  for (int j = 0; j < n_meta; ++j) l_i += fexp(meta[j] - m_i);

  f32x16 o[DP / 32];
#pragma unroll
  for (int t = 0; t < DP / 32; ++t) o[t] = zero16();

  const int klo = max(0, Q0 - W + 1) & ~31;
  const int khi = min(L, Q0 + 128);
  for (int k0 = klo; k0 < khi; k0 += 32) {
    __syncthreads();
    stage_rows<DP, true, false>(k + base, k0, L, d, kn, nullptr);
    stage_rows<DP, false, true>(v + base, k0, L, d, nullptr, vt);
    __syncthreads();
    if (q0 >= L || k0 > q0 + 31 || k0 + 31 < q0 - W + 1) continue;
    f32x16 s = zero16();
#pragma unroll
    for (int kb = 0; kb < DP / 16; ++kb) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(kn + col * T::NPITCH + 16 * kb + 8 * h);
      s = mfma(a, qreg[kb], s);
    }
    float mx = NEG_INF;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + acc_row(r, h);
      s[r] = in_window(qi, key, L, W) ? s[r] * scale : NEG_INF;
      mx = fmaxf(mx, s[r]);
    }
    mx = fmaxf(mx, xhalf(mx));
    const float m_new = fmaxf(m_i, mx);
    const float alpha = fexp(m_i - m_new);
    float ps = 0.f;
    bf16x8 p[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float e = fexp(s[r] - m_new);
      ps += e;
      p[r >> 3][r & 7] = to_bf16(e);
    }
    ps += xhalf(ps);
    l_i = l_i * alpha + ps;
#pragma unroll
    for (int t = 0; t < DP / 32; ++t) {
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= alpha;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(vt + (t * 32 + col) * T::TPITCH + 16 * kb + 8 * h);
        o[t] = mfma(a, p[kb], o[t]);
      }
    }
    m_i = m_new;
  }
  if (qi < L) {
    const float inv = 1.f / l_i;
#pragma unroll
    for (int t = 0; t < DP / 32; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g)
      {
        const int c = t * 32 + 8 * g + 4 * h;
        store4<bf16>(y + base, qi, c, d, o[t][4 * g] * inv, o[t][4 * g + 1] * inv,
                     o[t][4 * g + 2] * inv, o[t][4 * g + 3] * inv);
        if (y32)
          store4<float>(y32 + base, qi, c, d, o[t][4 * g] * inv, o[t][4 * g + 1] * inv,
                        o[t][4 * g + 2] * inv, o[t][4 * g + 3] * inv);
      }
    if (h == 0) lse[(size_t)bh * L + qi] = m_i + flog(l_i);
  }
}

// ----------------------------------------------------------------------------
// backward: grid (2*ceil(L/128), BH), 256 threads.  Blocks [0, NB) compute dq
// (and the per-block dmeta partial), blocks [NB, 2NB) compute dk and dv.
// ----------------------------------------------------------------------------
template <int DP, typename OutT>
__global__ __launch_bounds__(256) void swa_bwd_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ meta, int n_meta, const float* __restrict__ y32,
    const float* __restrict__ lse, const bf16* __restrict__ dy, OutT* __restrict__ dq,
    OutT* __restrict__ dk, OutT* __restrict__ dv, float* __restrict__ dmeta_part, int L, int d,
    int W, float scale) {
  using T = SwaTiles<DP>;
  extern __shared__ __align__(16) char smem[];
  bf16* nat0 = reinterpret_cast<bf16*>(smem);
  bf16* nat1 = nat0 + T::NAT_ELEMS;
  bf16* tr0 = nat1 + T::NAT_ELEMS;
  bf16* tr1 = tr0 + T::TR_ELEMS;
  float* rowv = reinterpret_cast<float*>(tr1 + T::TR_ELEMS);   // [2][32] lse, delta
  float* red = rowv + 64;                                       // [4][SWA_MAX_META]

  const int NB = (L + 127) / 128;
  const int bh = blockIdx.y;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int col = lane & 31, h = lane >> 5;
  const size_t base = (size_t)bh * L * d;

  if ((int)blockIdx.x < NB) {
    // ---------------- dq role: this wave owns queries q0..q0+31 ----------------
    const int Q0 = blockIdx.x * 128;
    const int q0 = Q0 + wave * 32;
    const int qi = q0 + col;
    bf16x8 qreg[DP / 16], dyreg[DP / 16];
    load_rows_operand<DP>(q + base, qi, L, d, h, qreg);
    load_rows_operand<DP>(dy + base, qi, L, d, h, dyreg);
    // delta = dy . y32 over this lane's k-slots (columns 16kb + 8(j/4) + 4h + j%4)
    float delta = 0.f;
    if (qi < L) {
      const float* yr = y32 + base + (size_t)qi * d;
#pragma unroll
      for (int kb = 0; kb < DP / 16; ++kb)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int c = 16 * kb + 8 * (j >> 2) + 4 * h + (j & 3);
          if (c < d) delta += to_f32(dyreg[kb][j]) * yr[c];
        }
    }
    delta += xhalf(delta);
    const float lse_i = qi < L ? lse[(size_t)bh * L + qi] : 0.f;

    f32x16 dqa[DP / 32];
#pragma unroll
    for (int t = 0; t < DP / 32; ++t) dqa[t] = zero16();

    const int klo = max(0, Q0 - W + 1) & ~31;
    const int khi = min(L, Q0 + 128);
    for (int k0 = klo; k0 < khi; k0 += 32) {
      __syncthreads();
      stage_rows<DP, true, true>(k + base, k0, L, d, nat0, tr0);
      stage_rows<DP, true, false>(v + base, k0, L, d, nat1, nullptr);
      __syncthreads();
      if (q0 >= L || k0 > q0 + 31 || k0 + 31 < q0 - W + 1) continue;
      f32x16 s = zero16(), dp = zero16();
#pragma unroll
      for (int kb = 0; kb < DP / 16; ++kb) {
        const bf16x8 ka = *reinterpret_cast<const bf16x8*>(nat0 + col * T::NPITCH + 16 * kb + 8 * h);
        const bf16x8 va = *reinterpret_cast<const bf16x8*>(nat1 + col * T::NPITCH + 16 * kb + 8 * h);
        s = mfma(ka, qreg[kb], s);
        dp = mfma(va, dyreg[kb], dp);
      }
      bf16x8 ds[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + acc_row(r, h);
        const float p = in_window(qi, key, L, W) ? fexp(s[r] * scale - lse_i) : 0.f;
        ds[r >> 3][r & 7] = to_bf16(p * (dp[r] - delta));
      }
#pragma unroll
      for (int t = 0; t < DP / 32; ++t)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          const bf16x8 a = *reinterpret_cast<const bf16x8*>(tr0 + (t * 32 + col) * T::TPITCH + 16 * kb + 8 * h);
          dqa[t] = mfma(a, ds[kb], dqa[t]);
        }
    }
    if (qi < L) {
#pragma unroll
      for (int t = 0; t < DP / 32; ++t)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          store4<OutT>(dq + base, qi, t * 32 + 8 * g + 4 * h, d, dqa[t][4 * g] * scale,
                       dqa[t][4 * g + 1] * scale, dqa[t][4 * g + 2] * scale,
                       dqa[t][4 * g + 3] * scale);
    }
    // dmeta partial of this block: -sum_i e^{meta_j - lse_i} delta_i
    for (int j = 0; j < n_meta; ++j) {
      float c = (qi < L && h == 0) ? fexp(meta[j] - lse_i) * delta : 0.f;
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) c += __shfl_xor(c, off);
      if (lane == 0) red[wave * SWA_MAX_META + j] = c;
    }
    __syncthreads();
    if ((int)threadIdx.x < n_meta) {
      const int j = threadIdx.x;
      const float c = red[j] + red[SWA_MAX_META + j] + red[2 * SWA_MAX_META + j] +
                      red[3 * SWA_MAX_META + j];
      dmeta_part[((size_t)bh * NB + blockIdx.x) * n_meta + j] = -c;
    }
    return;
  }

  // ---------------- dk/dv role: this wave owns keys kk0..kk0+31 ----------------
  const int K0 = (blockIdx.x - NB) * 128;
  const int kk0 = K0 + wave * 32;
  const int ti = kk0 + col;
  bf16x8 kreg[DP / 16], vreg[DP / 16];
  load_rows_operand<DP>(k + base, ti, L, d, h, kreg);
  load_rows_operand<DP>(v + base, ti, L, d, h, vreg);
  f32x16 dka[DP / 32], dva[DP / 32];
#pragma unroll
  for (int t = 0; t < DP / 32; ++t) {
    dka[t] = zero16();
    dva[t] = zero16();
  }
  const int qhi = min(L, K0 + 127 + W);
  for (int qq0 = K0; qq0 < qhi; qq0 += 32) {
    __syncthreads();
    stage_rows<DP, true, true>(q + base, qq0, L, d, nat0, tr0);
    stage_rows<DP, true, true>(dy + base, qq0, L, d, nat1, tr1);
    {
      // lse and delta of the 32 staged queries: 8 threads per query
      const int r = threadIdx.x >> 3, part = threadIdx.x & 7;
      const int qrow = qq0 + r;
      float acc = 0.f;
      if (qrow < L) {
        const float* yr = y32 + base + (size_t)qrow * d;
        const bf16* dr = dy + base + (size_t)qrow * d;
        for (int c = part; c < d; c += 8) acc += yr[c] * to_f32(dr[c]);
      }
      acc += __shfl_xor(acc, 1);
      acc += __shfl_xor(acc, 2);
      acc += __shfl_xor(acc, 4);
      if (part == 0) {
        rowv[r] = qrow < L ? lse[(size_t)bh * L + qrow] : 0.f;
        rowv[32 + r] = acc;
      }
    }
    __syncthreads();
    if (kk0 >= L || qq0 + 31 < kk0 || qq0 > kk0 + 31 + W - 1) continue;
    f32x16 s = zero16(), dp = zero16();
#pragma unroll
    for (int kb = 0; kb < DP / 16; ++kb) {
      const bf16x8 qa = *reinterpret_cast<const bf16x8*>(nat0 + col * T::NPITCH + 16 * kb + 8 * h);
      const bf16x8 da = *reinterpret_cast<const bf16x8*>(nat1 + col * T::NPITCH + 16 * kb + 8 * h);
      s = mfma(qa, kreg[kb], s);
      dp = mfma(da, vreg[kb], dp);
    }
    // s, dp: lane owns key ti, register r owns query qq0 + acc_row(r, h)
    bf16x8 pb[2], dsb[2];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qr = acc_row(r, h);
      const int qrow = qq0 + qr;
      const float p = in_window(qrow, ti, L, W) ? fexp(s[r] * scale - rowv[qr]) : 0.f;
      pb[r >> 3][r & 7] = to_bf16(p);
      dsb[r >> 3][r & 7] = to_bf16(p * (dp[r] - rowv[32 + qr]));
    }
#pragma unroll
    for (int t = 0; t < DP / 32; ++t)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const bf16x8 qa = *reinterpret_cast<const bf16x8*>(tr0 + (t * 32 + col) * T::TPITCH + 16 * kb + 8 * h);
        const bf16x8 da = *reinterpret_cast<const bf16x8*>(tr1 + (t * 32 + col) * T::TPITCH + 16 * kb + 8 * h);
        dva[t] = mfma(da, pb[kb], dva[t]);
        dka[t] = mfma(qa, dsb[kb], dka[t]);
      }
  }
  if (ti < L) {
#pragma unroll
    for (int t = 0; t < DP / 32; ++t)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int c = t * 32 + 8 * g + 4 * h;
        store4<OutT>(dk + base, ti, c, d, dka[t][4 * g] * scale, dka[t][4 * g + 1] * scale,
                     dka[t][4 * g + 2] * scale, dka[t][4 * g + 3] * scale);
        store4<OutT>(dv + base, ti, c, d, dva[t][4 * g], dva[t][4 * g + 1], dva[t][4 * g + 2],
                     dva[t][4 * g + 3]);
      }
  }
}

// ----------------------------------------------------------------------------
// host launchers
// ----------------------------------------------------------------------------
template <int DP>
static size_t swa_fwd_lds() {
  return (SwaTiles<DP>::NAT_ELEMS + SwaTiles<DP>::TR_ELEMS) * sizeof(bf16);
}
template <int DP>
static size_t swa_bwd_lds() {
  return (2 * SwaTiles<DP>::NAT_ELEMS + 2 * SwaTiles<DP>::TR_ELEMS) * sizeof(bf16) +
         (64 + 4 * SWA_MAX_META) * sizeof(float);
}

template <int DP>
static hipError_t launch_swa_fwd_t(const void* q, const void* k, const void* v, const float* meta,
                                   int n_meta, void* y, float* y32, float* lse, int BH, int L,
                                   int d, int W, float scale, hipStream_t st) {
  const size_t lds = swa_fwd_lds<DP>();
  auto kern = swa_fwd_kernel<DP>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  dim3 grid((L + 127) / 128, BH);
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, (const bf16*)q, (const bf16*)k,
                     (const bf16*)v, meta, n_meta, (bf16*)y, y32, lse, L, d, W, scale);
  return hipGetLastError();
}

template <int DP, typename OutT>
static hipError_t launch_swa_bwd_t(const void* q, const void* k, const void* v, const float* meta,
                                   int n_meta, const float* y32, const float* lse, const void* dy,
                                   void* dq, void* dk, void* dv, float* dmeta_part, int BH, int L,
                                   int d, int W, float scale, hipStream_t st) {
  const size_t lds = swa_bwd_lds<DP>();
  auto kern = swa_bwd_kernel<DP, OutT>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  const int NB = (L + 127) / 128;
  dim3 grid(2 * NB, BH);
  hipLaunchKernelGGL(kern, grid, dim3(256), lds, st, (const bf16*)q, (const bf16*)k,
                     (const bf16*)v, meta, n_meta, y32, lse, (const bf16*)dy,
                     (OutT*)dq, (OutT*)dk, (OutT*)dv, dmeta_part, L, d, W, scale);
  return hipGetLastError();
}

int swa_padded_dim(int d) {
  if (d <= 32) return 32;
  if (d <= 64) return 64;
  if (d <= 128) return 128;
  if (d <= 256) return 256;
  return -1;
}

hipError_t launch_swa_fwd(const void* q, const void* k, const void* v, const float* meta,
                          int n_meta, void* y, float* y32, float* lse, int BH, int L, int d, int W,
                          float scale, hipStream_t st) {
  switch (swa_padded_dim(d)) {
    case 32: return launch_swa_fwd_t<32>(q, k, v, meta, n_meta, y, y32, lse, BH, L, d, W, scale, st);
    case 64: return launch_swa_fwd_t<64>(q, k, v, meta, n_meta, y, y32, lse, BH, L, d, W, scale, st);
    case 128: return launch_swa_fwd_t<128>(q, k, v, meta, n_meta, y, y32, lse, BH, L, d, W, scale, st);
    case 256: return launch_swa_fwd_t<256>(q, k, v, meta, n_meta, y, y32, lse, BH, L, d, W, scale, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_swa_bwd(const void* q, const void* k, const void* v, const float* meta,
                          int n_meta, const float* y32, const float* lse, const void* dy, void* dq,
                          void* dk, void* dv, bool grad_bf16, float* dmeta_part, int BH, int L,
                          int d, int W, float scale, hipStream_t st) {
#define LZ_SWA_BWD(DPV)                                                                      \
  return grad_bf16 ? launch_swa_bwd_t<DPV, bf16>(q, k, v, meta, n_meta, y32, lse, dy, dq, dk, \
                                                 dv, dmeta_part, BH, L, d, W, scale, st)     \
                   : launch_swa_bwd_t<DPV, float>(q, k, v, meta, n_meta, y32, lse, dy, dq, dk, \
                                                  dv, dmeta_part, BH, L, d, W, scale, st)
  switch (swa_padded_dim(d)) {
    case 32: LZ_SWA_BWD(32);
    case 64: LZ_SWA_BWD(64);
    case 128: LZ_SWA_BWD(128);
    case 256: LZ_SWA_BWD(256);
    default: return hipErrorInvalidValue;
  }
#undef LZ_SWA_BWD
}

}  // namespace lz
