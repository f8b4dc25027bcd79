// Chunked gated linear attention, backward, for gfx950.
//
// Reference: _GLA.backward and its kernels (src/kernels/gla.py:104-194,
// 236-256), with the autograd steps of the gate path (gla.py:260-262).  With
// the chunk-local notation of gla_fwd.hip (lg, qs = e^{lg}, ks = e^{lg_end-lg},
// r = e^{lg_end}, decay_it = e^{lg_i - lg_t}) and the forward state S_n, z_n:
//   delta_i = dy_i . y_i                              (fp32 y)
//   dA_it   = [t<=i] (dy_i . v_t - delta_i) / den_i,  dad = dA * decay
//   dfq_i   = sum_t dad_it fk_t + (qs_i/den_i) (dy_i S_n^T - delta_i z_n)
//   dfk_t   = sum_i dad_it fq_i + ks_t (v_t dS_n^T - dz_n)
//   dv_t    = sum_i (a_it/den_i) dy_i + K~_t dS_n
//   dS_n    = r_{n+1} dS_{n+1} + Q^_{n+1}^T dY_{n+1},  Q^_i = bf16(fq_i qs_i / den_i)
//   dz_n    = r_{n+1} dz_{n+1} + sum_i Q^_i delta_i
//   dG_j    = fq_j . dfq_j - fk_j . dfk_j,  d log_gamma = reverse cumsum of dG
//             (summed over heads for a per-token gate)
//
// Three launches, none of which writes a state to HBM:
//   A (forward walk, one workgroup per (b,h)): carries S^T (d x f) in MFMA
//     accumulators; recomputes den and delta -- delta_i = dy_i . o_i / den_i
//     with dy_i . o_i = Q~_i . (S_n dy_i) + sum_t a_it (v_t . dy_i), both
//     products it needs anyway -- and writes dfq, den, delta and fq.dfq.
//   B (reverse walk, one workgroup per (b,h)): carries dS (f x d) and dS^T
//     (d x f) in accumulators (dv contracts the state over f, dfk over d, and
//     an accumulator can only be contracted over its rows); writes dv, dfk and
//     dG.
//   G: d log_gamma = reverse cumsum of dG (head-summed for per-token gates).
#include "common.hpp"

namespace lz {

constexpr int GC = 64;   // chunk length

// Stage rows [t0, t0+64) of a [L x ncols] matrix: natural tile (slot order
// along the columns) and/or transposed tile (slot order along the tokens).
template <int KP>
__device__ __forceinline__ void stage_chunk(const bf16* __restrict__ src, int t0, int L, int ncols,
                                            bf16* nat, int npitch, bf16* tr, int tpitch) {
  constexpr int K4 = KP / 4;
  for (int idx = threadIdx.x; idx < GC * K4; idx += 256) {
    const int r = idx / K4, c = (idx % K4) * 4;
    const bf16x4 x = load4(src, t0 + r, c, L, ncols);
    if (nat) *reinterpret_cast<bf16x4*>(nat + r * npitch + pidx(c)) = x;
    if (tr) {
#pragma unroll
      for (int e = 0; e < 4; ++e) tr[(c + e) * tpitch + pidx(r)] = x[e];
    }
  }
}

// Chunk-local inclusive scan of the gate by one wave; writes lg[64],
// e^{lg}[64] (natural order), e^{end-lg} in slot order, and e^{end}.
__device__ __forceinline__ void scan_gate(const float* __restrict__ lgb, int t0, int L, int lane,
                                          float* lgs, float* qs, float* kss, float* rdec) {
  float g = (t0 + lane < L) ? lgb[t0 + lane] : 0.f;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float o = __shfl_up(g, off);
    if (lane >= off) g += o;
  }
  const float end = __shfl(g, 63);
  lgs[lane] = g;
  qs[lane] = fexp(g);
  kss[pidx(lane)] = fexp(end - g);
  if (lane == 0) rdec[0] = fexp(end);
}

// Which 32-wide tiles of a dimension with NT32 tiles a wave owns, and which
// 32-token halves of the chunk it pairs them with.  Every (tile, half) pair
// has exactly one owner; with fewer than 4 tiles a tile is owned by two waves
// (one per half), which then both keep that tile's state.
template <int NT32>
struct Own {
  static constexpr int TILES = NT32 >= 4 ? NT32 / 4 : 1;
  static constexpr int HALVES = NT32 >= 4 ? 2 : 1;
  __device__ static bool active(int wave) { return NT32 >= 2 || wave < 2; }
  __device__ static int tile(int wave, int i) {
    return NT32 >= 4 ? wave + 4 * i : (NT32 == 2 ? (wave >> 1) : 0);
  }
  __device__ static int half(int wave, int j) { return NT32 >= 4 ? j : (wave & 1); }
};

// ----------------------------------------------------------------------------
// kernel A: forward walk -> dfq, den, delta, p = fq . dfq
// ----------------------------------------------------------------------------
template <int FP, int DP>
struct BwdACfg {
  static constexpr int NPF = FP + 8, NPD = DP + 8, TP = GC + 8;
  static constexpr int OFF_FQN = 0;
  static constexpr int OFF_FKN = OFF_FQN + GC * NPF * 2;
  static constexpr int OFF_FKT = OFF_FKN + GC * NPF * 2;
  static constexpr int OFF_VN = OFF_FKT + FP * TP * 2;
  static constexpr int OFF_VT = OFF_VN + GC * NPD * 2;
  static constexpr int OFF_DYN = OFF_VT + DP * TP * 2;
  static constexpr int OFF_FR = OFF_DYN + GC * NPD * 2;          // dad fragments [2][4][64] bf16x8
  static constexpr int OFF_RA = OFF_FR + 2 * 4 * 64 * 16;         // [2][64] sum_t a
  static constexpr int OFF_RAV = OFF_RA + 2 * 64 * 4;             // [2][64] sum_t a (v.dy)
  static constexpr int OFF_QZ = OFF_RAV + 2 * 64 * 4;             // [4][64] Q~.z partials
  static constexpr int OFF_NX = OFF_QZ + 4 * 64 * 4;              // [8][64] Q~.(S dy) partials
  static constexpr int OFF_PP = OFF_NX + 8 * 64 * 4;              // [8][64] fq.dfq partials
  static constexpr int OFF_DEN = OFF_PP + 8 * 64 * 4;             // [64]
  static constexpr int OFF_DEL = OFF_DEN + 64 * 4;                // [64]
  static constexpr int OFF_LG = OFF_DEL + 64 * 4;
  static constexpr int OFF_QS = OFF_LG + 64 * 4;
  static constexpr int OFF_KS = OFF_QS + 64 * 4;
  static constexpr int OFF_Z = OFF_KS + 64 * 4;                   // [FP] natural order
  static constexpr int OFF_R = OFF_Z + FP * 4;
  static constexpr int BYTES = OFF_R + 16;
};

template <int FP, int DP, typename OutT>
__global__ __launch_bounds__(256) void gla_bwd_a_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, const bf16* __restrict__ dy, OutT* __restrict__ dfq,
    float* __restrict__ den_out, float* __restrict__ delta_out, float* __restrict__ p_out, int H,
    int L, int F, int D, int gate_per_head) {
  using Cfg = BwdACfg<FP, DP>;
  constexpr int NPF = Cfg::NPF, NPD = Cfg::NPD, TP = Cfg::TP;
  constexpr int NFT = FP / 32, NDT = DP / 32;
  using OF = Own<NFT>;
  extern __shared__ __align__(16) char smem[];
  bf16* fqn = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQN);
  bf16* fkn = reinterpret_cast<bf16*>(smem + Cfg::OFF_FKN);
  bf16* fkt = reinterpret_cast<bf16*>(smem + Cfg::OFF_FKT);
  bf16* vn = reinterpret_cast<bf16*>(smem + Cfg::OFF_VN);
  bf16* vt = reinterpret_cast<bf16*>(smem + Cfg::OFF_VT);
  bf16* dyn = reinterpret_cast<bf16*>(smem + Cfg::OFF_DYN);
  bf16x8* fr = reinterpret_cast<bf16x8*>(smem + Cfg::OFF_FR);
  float* ra = reinterpret_cast<float*>(smem + Cfg::OFF_RA);
  float* rav = reinterpret_cast<float*>(smem + Cfg::OFF_RAV);
  float* qz = reinterpret_cast<float*>(smem + Cfg::OFF_QZ);
  float* nx = reinterpret_cast<float*>(smem + Cfg::OFF_NX);
  float* pp = reinterpret_cast<float*>(smem + Cfg::OFF_PP);
  float* dens = reinterpret_cast<float*>(smem + Cfg::OFF_DEN);
  float* dels = reinterpret_cast<float*>(smem + Cfg::OFF_DEL);
  float* lgs = reinterpret_cast<float*>(smem + Cfg::OFF_LG);
  float* qs = reinterpret_cast<float*>(smem + Cfg::OFF_QS);
  float* kss = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  float* zs = reinterpret_cast<float*>(smem + Cfg::OFF_Z);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  const int bh = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const size_t offF = (size_t)bh * L * F, offD = (size_t)bh * L * D, offL = (size_t)bh * L;
  const float* lgb = log_gamma + (size_t)(gate_per_head ? bh : bh / H) * L;

  for (int f = tid; f < FP; f += 256) zs[f] = 0.f;

  // S^T[d-tile][owned f-tile]: rows d, cols f
  f32x16 St[NDT][OF::TILES];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < OF::TILES; ++i) St[dt][i] = zero16();

  const int kt = wave >> 1, qt = wave & 1;   // this wave's tile of the 64x64 score block
  const int qi = qt * 32 + col;               // chunk-local query of this lane
  const int NT = (L + GC - 1) / GC;
  for (int n = 0; n < NT; ++n) {
    const int t0 = n * GC;
    __syncthreads();
    if (n > 0 && tid < 64 && t0 - GC + tid < L) {   // fq.dfq of the previous chunk
      float s = 0.f;
      for (int ft = 0; ft < NFT; ++ft) s += pp[ft * 64 + tid];
      p_out[offL + t0 - GC + tid] = s;
    }
    stage_chunk<FP>(fq + offF, t0, L, F, fqn, NPF, nullptr, 0);
    stage_chunk<FP>(fk + offF, t0, L, F, fkn, NPF, fkt, TP);
    stage_chunk<DP>(v + offD, t0, L, D, vn, NPD, vt, TP);
    stage_chunk<DP>(dy + offD, t0, L, D, dyn, NPD, nullptr, 0);
    if (wave == 0) scan_gate(lgb, t0, L, lane, lgs, qs, kss, rdec);
    __syncthreads();

    // ---- P1: a^T and (v dy^T) tile of this wave; X = S dy^T ----------------
    f32x16 aT = zero16(), vdy = zero16();
#pragma unroll
    for (int kb = 0; kb < FP / 16; ++kb) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(fkn + (kt * 32 + col) * NPF + 16 * kb + 8 * h);
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(fqn + qi * NPF + 16 * kb + 8 * h);
      aT = mfma(a, b, aT);
    }
#pragma unroll
    for (int kb = 0; kb < DP / 16; ++kb) {
      const bf16x8 a = *reinterpret_cast<const bf16x8*>(vn + (kt * 32 + col) * NPD + 16 * kb + 8 * h);
      const bf16x8 b = *reinterpret_cast<const bf16x8*>(dyn + qi * NPD + 16 * kb + 8 * h);
      vdy = mfma(a, b, vdy);
    }
    const float lgq = lgs[qi];
    {
      float sa = 0.f, sav = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt * 32 + acc_row(r, h);
        const float dec = key <= qi ? fexp(lgq - lgs[key]) : 0.f;
        aT[r] = to_f32(to_bf16(aT[r] * dec));   // a exactly as the forward rounds it
        sa += aT[r];
        sav += aT[r] * vdy[r];
      }
      sa += xhalf(sa);
      sav += xhalf(sav);
      if (h == 0) {
        ra[kt * 64 + qi] = sa;
        rav[kt * 64 + qi] = sav;
      }
      constexpr int FQ = FP / 4;   // Q~ . z over a quarter of the features, query = lane
      const float qsv = qs[lane];
      float acc = 0.f;
      for (int fs = wave * FQ; fs < (wave + 1) * FQ; ++fs)
        acc += to_f32(to_bf16(to_f32(fqn[lane * NPF + fs]) * qsv)) * zs[pidx(fs)];
      qz[wave * 64 + lane] = acc;
    }
    f32x16 X[OF::TILES][OF::HALVES];
    if (OF::active(wave)) {
#pragma unroll
      for (int i = 0; i < OF::TILES; ++i) {
        const int ft = OF::tile(wave, i);
#pragma unroll
        for (int j = 0; j < OF::HALVES; ++j) {
          const int q = OF::half(wave, j) * 32 + col;
          f32x16 x = zero16();
#pragma unroll
          for (int kb = 0; kb < DP / 16; ++kb) {
            const bf16x8 b = *reinterpret_cast<const bf16x8*>(dyn + q * NPD + 16 * kb + 8 * h);
            x = mfma(acc_operand(St[kb >> 1][i], kb & 1), b, x);
          }
          X[i][j] = x;
          const float qsv = qs[q];
          float s = 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int f = ft * 32 + acc_row(r, h);
            s += to_f32(to_bf16(to_f32(fqn[q * NPF + pidx(f)]) * qsv)) * x[r];
          }
          s += xhalf(s);
          if (h == 0) nx[ft * 64 + q] = s;
        }
      }
    }
    __syncthreads();

    // ---- P2: den, delta and dad fragments -----------------------------------
    {
      const float den = ra[qi] + ra[64 + qi] + qz[qi] + qz[64 + qi] + qz[128 + qi] + qz[192 + qi];
      float num = rav[qi] + rav[64 + qi];
      for (int ft = 0; ft < NFT; ++ft) num += nx[ft * 64 + qi];
      const float dcl = fmaxf(den, TINY);
      const float delta = num / dcl;
      const float inv = 1.f / dcl;
      bf16x8 d8[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt * 32 + acc_row(r, h);
        const float dec = key <= qi ? fexp(lgq - lgs[key]) : 0.f;
        d8[r >> 3][r & 7] = to_bf16((vdy[r] - delta) * inv * dec);
      }
      fr[(qt * 4 + kt * 2 + 0) * 64 + lane] = d8[0];
      fr[(qt * 4 + kt * 2 + 1) * 64 + lane] = d8[1];
      if (kt == 0 && h == 0) {
        dens[qi] = den;
        dels[qi] = delta;
        if (t0 + qi < L) {
          den_out[offL + t0 + qi] = den;
          delta_out[offL + t0 + qi] = delta;
        }
      }
    }
    __syncthreads();

    // ---- P3: dfq for owned (f-tile, half); S^T and z update -----------------
    const float r_n = rdec[0];
    if (OF::active(wave)) {
#pragma unroll
      for (int i = 0; i < OF::TILES; ++i) {
        const int ft = OF::tile(wave, i);
#pragma unroll
        for (int j = 0; j < OF::HALVES; ++j) {
          const int hq = OF::half(wave, j);
          const int q = hq * 32 + col;
          f32x16 g = zero16();
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(fkt + (ft * 32 + col) * TP + 16 * kb + 8 * h);
            g = mfma(a, fr[(hq * 4 + kb) * 64 + lane], g);
          }
          const float dcl = fmaxf(dens[q], TINY);
          const float qsd = qs[q] / dcl;
          const float delta = dels[q];
          const int tok = t0 + q;
          float ps = 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int f = ft * 32 + acc_row(r, h);
            g[r] += qsd * (X[i][j][r] - zs[f] * delta);
            ps += to_f32(fqn[q * NPF + pidx(f)]) * g[r];
          }
          ps += xhalf(ps);
          if (h == 0) pp[ft * 64 + q] = tok < L ? ps : 0.f;
          if (tok < L) {
#pragma unroll
            for (int gg = 0; gg < 4; ++gg)
              store4<OutT>(dfq + offF, tok, ft * 32 + 8 * gg + 4 * h, F, g[4 * gg],
                           g[4 * gg + 1], g[4 * gg + 2], g[4 * gg + 3]);
          }
        }
        // S^T[:, ft] <- r S^T + V^T K~
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) St[dt][i][r] *= r_n;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(vt + (dt * 32 + col) * TP + 16 * kb + 8 * h);
            const bf16x8 raw = *reinterpret_cast<const bf16x8*>(fkt + (ft * 32 + col) * TP + 16 * kb + 8 * h);
            bf16x8 b;
#pragma unroll
            for (int e = 0; e < 8; ++e) b[e] = to_bf16(to_f32(raw[e]) * kss[16 * kb + 8 * h + e]);
            St[dt][i] = mfma(a, b, St[dt][i]);
          }
        }
      }
    }
    __syncthreads();   // z is read above (P3) before it is updated
    for (int f = tid; f < FP; f += 256) {
      float acc = 0.f;
      for (int t = 0; t < GC; ++t) acc += to_f32(to_bf16(to_f32(fkt[f * TP + t]) * kss[t]));
      zs[f] = zs[f] * r_n + acc;
    }
  }
  __syncthreads();
  {
    const int t0 = (NT - 1) * GC;
    if (tid < 64 && t0 + tid < L) {
      float s = 0.f;
      for (int ft = 0; ft < NFT; ++ft) s += pp[ft * 64 + tid];
      p_out[offL + t0 + tid] = s;
    }
  }
}

// ----------------------------------------------------------------------------
// kernel B: reverse walk -> dv, dfk, dG = p - fk . dfk
// ----------------------------------------------------------------------------
template <int FP, int DP>
struct BwdBCfg {
  static constexpr int NPF = FP + 8, NPD = DP + 8, TP = GC + 8;
  static constexpr int OFF_FQN = 0;
  static constexpr int OFF_FQT = OFF_FQN + GC * NPF * 2;
  static constexpr int OFF_FKN = OFF_FQT + FP * TP * 2;
  static constexpr int OFF_VN = OFF_FKN + GC * NPF * 2;
  static constexpr int OFF_DYN = OFF_VN + GC * NPD * 2;
  static constexpr int OFF_DYT = OFF_DYN + GC * NPD * 2;
  static constexpr int OFF_FA = OFF_DYT + DP * TP * 2;           // a/den fragments [2 kt][4 qb][64]
  static constexpr int OFF_FD = OFF_FA + 2 * 4 * 64 * 16;         // dad fragments
  static constexpr int OFF_PK = OFF_FD + 2 * 4 * 64 * 16;         // [8][64] fk.dfk partials
  static constexpr int OFF_DEN = OFF_PK + 8 * 64 * 4;             // [64] natural
  static constexpr int OFF_DEL = OFF_DEN + 64 * 4;                // [64] natural
  static constexpr int OFF_P = OFF_DEL + 64 * 4;                  // [64] fq.dfq
  static constexpr int OFF_QH = OFF_P + 64 * 4;                   // [64] e^{lg}/den, slot order
  static constexpr int OFF_LG = OFF_QH + 64 * 4;
  static constexpr int OFF_QS = OFF_LG + 64 * 4;
  static constexpr int OFF_KS = OFF_QS + 64 * 4;                  // slot order
  static constexpr int OFF_KSN = OFF_KS + 64 * 4;                 // natural order
  static constexpr int OFF_DZ = OFF_KSN + 64 * 4;                 // [2][FP] double-buffered dz
  static constexpr int OFF_R = OFF_DZ + 2 * FP * 4;
  static constexpr int BYTES = OFF_R + 16;
};

template <int FP, int DP, typename OutT>
__global__ __launch_bounds__(256) void gla_bwd_b_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, const bf16* __restrict__ dy,
    const float* __restrict__ den_in, const float* __restrict__ delta_in,
    const float* __restrict__ p_in, OutT* __restrict__ dfk, OutT* __restrict__ dv,
    float* __restrict__ dG, int H, int L, int F, int D, int gate_per_head) {
  using Cfg = BwdBCfg<FP, DP>;
  constexpr int NPF = Cfg::NPF, NPD = Cfg::NPD, TP = Cfg::TP;
  constexpr int NFT = FP / 32, NDT = DP / 32;
  using OF = Own<NFT>;
  using OD = Own<NDT>;
  extern __shared__ __align__(16) char smem[];
  bf16* fqn = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQN);
  bf16* fqt = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQT);
  bf16* fkn = reinterpret_cast<bf16*>(smem + Cfg::OFF_FKN);
  bf16* vn = reinterpret_cast<bf16*>(smem + Cfg::OFF_VN);
  bf16* dyn = reinterpret_cast<bf16*>(smem + Cfg::OFF_DYN);
  bf16* dyt = reinterpret_cast<bf16*>(smem + Cfg::OFF_DYT);
  bf16x8* fa = reinterpret_cast<bf16x8*>(smem + Cfg::OFF_FA);
  bf16x8* fd = reinterpret_cast<bf16x8*>(smem + Cfg::OFF_FD);
  float* pk = reinterpret_cast<float*>(smem + Cfg::OFF_PK);
  float* dens = reinterpret_cast<float*>(smem + Cfg::OFF_DEN);
  float* dels = reinterpret_cast<float*>(smem + Cfg::OFF_DEL);
  float* ps = reinterpret_cast<float*>(smem + Cfg::OFF_P);
  float* qhs = reinterpret_cast<float*>(smem + Cfg::OFF_QH);
  float* lgs = reinterpret_cast<float*>(smem + Cfg::OFF_LG);
  float* qs = reinterpret_cast<float*>(smem + Cfg::OFF_QS);
  float* kss = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  float* ksn = reinterpret_cast<float*>(smem + Cfg::OFF_KSN);
  float* dzs = reinterpret_cast<float*>(smem + Cfg::OFF_DZ);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  const int bh = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const size_t offF = (size_t)bh * L * F, offD = (size_t)bh * L * D, offL = (size_t)bh * L;
  const float* lgb = log_gamma + (size_t)(gate_per_head ? bh : bh / H) * L;

  for (int f = tid; f < 2 * FP; f += 256) dzs[f] = 0.f;

  // dS[f-tile][owned d-tile] (rows f, cols d); dS^T[d-tile][owned f-tile] (rows d, cols f)
  f32x16 dS[NFT][OD::TILES];
  f32x16 dSt[NDT][OF::TILES];
#pragma unroll
  for (int ft = 0; ft < NFT; ++ft)
#pragma unroll
    for (int i = 0; i < OD::TILES; ++i) dS[ft][i] = zero16();
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
    for (int i = 0; i < OF::TILES; ++i) dSt[dt][i] = zero16();

  const int qt = wave >> 1, kt = wave & 1;   // this wave's tile of the score block
  const int ki = kt * 32 + col;               // chunk-local key of this lane (P1)
  const int NT = (L + GC - 1) / GC;
  int cur = 0;                                 // dz buffer holding dz_n
  for (int n = NT - 1; n >= 0; --n) {
    const int t0 = n * GC;
    __syncthreads();
    stage_chunk<FP>(fq + offF, t0, L, F, fqn, NPF, fqt, TP);
    stage_chunk<FP>(fk + offF, t0, L, F, fkn, NPF, nullptr, 0);
    stage_chunk<DP>(v + offD, t0, L, D, vn, NPD, nullptr, 0);
    stage_chunk<DP>(dy + offD, t0, L, D, dyn, NPD, dyt, TP);
    if (wave == 0) scan_gate(lgb, t0, L, lane, lgs, qs, kss, rdec);
    if (wave == 1) {
      const bool ok = t0 + lane < L;
      const float den = ok ? fmaxf(den_in[offL + t0 + lane], TINY) : 1.f;
      dens[lane] = den;
      dels[lane] = ok ? delta_in[offL + t0 + lane] : 0.f;
      ps[lane] = ok ? p_in[offL + t0 + lane] : 0.f;
    }
    __syncthreads();
    if (tid < 64) {
      qhs[pidx(tid)] = qs[tid] / dens[tid];
      ksn[tid] = kss[pidx(tid)];
    }

    // ---- P1: s and (dy v^T) tile (queries x keys); a/den and dad fragments ----
    {
      f32x16 s = zero16(), dyv = zero16();
#pragma unroll
      for (int kb = 0; kb < FP / 16; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(fqn + (qt * 32 + col) * NPF + 16 * kb + 8 * h);
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(fkn + ki * NPF + 16 * kb + 8 * h);
        s = mfma(a, b, s);
      }
#pragma unroll
      for (int kb = 0; kb < DP / 16; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(dyn + (qt * 32 + col) * NPD + 16 * kb + 8 * h);
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(vn + ki * NPD + 16 * kb + 8 * h);
        dyv = mfma(a, b, dyv);
      }
      const float lgk = lgs[ki];
      bf16x8 fa8[2], fd8[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int q = qt * 32 + acc_row(r, h);
        const bool c = ki <= q;
        const float dec = c ? fexp(lgs[q] - lgk) : 0.f;
        const float den = dens[q];
        const float a = to_f32(to_bf16(s[r] * dec));
        fa8[r >> 3][r & 7] = to_bf16(a / den);
        fd8[r >> 3][r & 7] = to_bf16(c ? (dyv[r] - dels[q]) / den * dec : 0.f);
      }
      fa[(kt * 4 + qt * 2 + 0) * 64 + lane] = fa8[0];
      fa[(kt * 4 + qt * 2 + 1) * 64 + lane] = fa8[1];
      fd[(kt * 4 + qt * 2 + 0) * 64 + lane] = fd8[0];
      fd[(kt * 4 + qt * 2 + 1) * 64 + lane] = fd8[1];
    }
    __syncthreads();

    // ---- P2: dv (owned d-tiles), dfk (owned f-tiles), state updates ----------
    const float r_n = rdec[0];
    const float* dz = dzs + cur * FP;
    if (OD::active(wave)) {
#pragma unroll
      for (int i = 0; i < OD::TILES; ++i) {
        const int dt = OD::tile(wave, i);
#pragma unroll
        for (int j = 0; j < OD::HALVES; ++j) {
          const int hk = OD::half(wave, j);
          const int key = hk * 32 + col;
          const float ksv = ksn[key];
          f32x16 g = zero16();
#pragma unroll
          for (int qb = 0; qb < 4; ++qb) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(dyt + (dt * 32 + col) * TP + 16 * qb + 8 * h);
            g = mfma(a, fa[(hk * 4 + qb) * 64 + lane], g);
          }
#pragma unroll
          for (int kb = 0; kb < FP / 16; ++kb) {
            const bf16x8 raw = *reinterpret_cast<const bf16x8*>(fkn + key * NPF + 16 * kb + 8 * h);
            bf16x8 b;
#pragma unroll
            for (int e = 0; e < 8; ++e) b[e] = to_bf16(to_f32(raw[e]) * ksv);
            g = mfma(acc_operand(dS[kb >> 1][i], kb & 1), b, g);
          }
          const int tok = t0 + key;
          if (tok < L) {
#pragma unroll
            for (int gg = 0; gg < 4; ++gg)
              store4<OutT>(dv + offD, tok, dt * 32 + 8 * gg + 4 * h, D, g[4 * gg],
                           g[4 * gg + 1], g[4 * gg + 2], g[4 * gg + 3]);
          }
        }
      }
    }
    if (OF::active(wave)) {
#pragma unroll
      for (int i = 0; i < OF::TILES; ++i) {
        const int ft = OF::tile(wave, i);
#pragma unroll
        for (int j = 0; j < OF::HALVES; ++j) {
          const int hk = OF::half(wave, j);
          const int key = hk * 32 + col;
          f32x16 x = zero16();
#pragma unroll
          for (int kb = 0; kb < DP / 16; ++kb) {
            const bf16x8 b = *reinterpret_cast<const bf16x8*>(vn + key * NPD + 16 * kb + 8 * h);
            x = mfma(acc_operand(dSt[kb >> 1][i], kb & 1), b, x);
          }
          f32x16 g = zero16();
#pragma unroll
          for (int qb = 0; qb < 4; ++qb) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(fqt + (ft * 32 + col) * TP + 16 * qb + 8 * h);
            g = mfma(a, fd[(hk * 4 + qb) * 64 + lane], g);
          }
          const float ksv = ksn[key];
          const int tok = t0 + key;
          float pks = 0.f;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int f = ft * 32 + acc_row(r, h);
            g[r] += ksv * (x[r] - dz[f]);
            pks += to_f32(fkn[key * NPF + pidx(f)]) * g[r];
          }
          pks += xhalf(pks);
          if (h == 0) pk[ft * 64 + key] = pks;
          if (tok < L) {
#pragma unroll
            for (int gg = 0; gg < 4; ++gg)
              store4<OutT>(dfk + offF, tok, ft * 32 + 8 * gg + 4 * h, F, g[4 * gg],
                           g[4 * gg + 1], g[4 * gg + 2], g[4 * gg + 3]);
          }
        }
      }
    }
    // dS <- r dS + Q^^T dY ; dS^T <- r dS^T + dY^T Q^   (after this chunk used them)
    if (OD::active(wave)) {
#pragma unroll
      for (int i = 0; i < OD::TILES; ++i) {
        const int dt = OD::tile(wave, i);
#pragma unroll
        for (int ft = 0; ft < NFT; ++ft) {
#pragma unroll
          for (int r = 0; r < 16; ++r) dS[ft][i][r] *= r_n;
#pragma unroll
          for (int qb = 0; qb < 4; ++qb) {
            const bf16x8 raw = *reinterpret_cast<const bf16x8*>(fqt + (ft * 32 + col) * TP + 16 * qb + 8 * h);
            bf16x8 a;
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = to_bf16(to_f32(raw[e]) * qhs[16 * qb + 8 * h + e]);
            const bf16x8 b = *reinterpret_cast<const bf16x8*>(dyt + (dt * 32 + col) * TP + 16 * qb + 8 * h);
            dS[ft][i] = mfma(a, b, dS[ft][i]);
          }
        }
      }
    }
    if (OF::active(wave)) {
#pragma unroll
      for (int i = 0; i < OF::TILES; ++i) {
        const int ft = OF::tile(wave, i);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
          for (int r = 0; r < 16; ++r) dSt[dt][i][r] *= r_n;
#pragma unroll
          for (int qb = 0; qb < 4; ++qb) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(dyt + (dt * 32 + col) * TP + 16 * qb + 8 * h);
            const bf16x8 raw = *reinterpret_cast<const bf16x8*>(fqt + (ft * 32 + col) * TP + 16 * qb + 8 * h);
            bf16x8 b;
#pragma unroll
            for (int e = 0; e < 8; ++e) b[e] = to_bf16(to_f32(raw[e]) * qhs[16 * qb + 8 * h + e]);
            dSt[dt][i] = mfma(a, b, dSt[dt][i]);
          }
        }
      }
    }
    // dz_{n-1} = r dz_n + sum_i Q^_i delta_i  into the other buffer
    for (int f = tid; f < FP; f += 256) {
      float acc = 0.f;
      for (int t = 0; t < GC; ++t)
        acc += to_f32(to_bf16(to_f32(fqt[f * TP + t]) * qhs[t])) * dels[pidx(t)];
      dzs[(cur ^ 1) * FP + f] = dz[f] * r_n + acc;
    }
    __syncthreads();
    if (tid < 64 && t0 + tid < L) {
      float s = 0.f;
      for (int ft = 0; ft < NFT; ++ft) s += pk[ft * 64 + tid];
      dG[offL + t0 + tid] = ps[tid] - s;
    }
    cur ^= 1;
  }
}

// ----------------------------------------------------------------------------
// kernel G: d log_gamma[row, j] = sum_{j' >= j} value[row, j'], where value is
// dG of that (b, h) row (per-head gate) or its sum over heads (per-token gate).
// One workgroup per output row; deterministic order.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gla_gate_grad_kernel(const float* __restrict__ dG,
                                                            float* __restrict__ dlg, int H, int L,
                                                            int gate_per_head) {
  __shared__ float tot[256];
  const int row = blockIdx.x, tid = threadIdx.x;
  const int nsum = gate_per_head ? 1 : H;
  const float* src = dG + (size_t)row * nsum * L;
  const int seg = (L + 255) / 256;
  const int lo = min(L, tid * seg), hi = min(L, lo + seg);
  auto value = [&](int j) {
    float s = 0.f;
    for (int hh = 0; hh < nsum; ++hh) s += src[(size_t)hh * L + j];
    return s;
  };
  float t = 0.f;
  for (int j = hi - 1; j >= lo; --j) t += value(j);
  tot[tid] = t;
  __syncthreads();
  if (tid == 0) {
    float acc = 0.f;
    for (int i = 255; i >= 0; --i) {
      const float x = tot[i];
      tot[i] = acc;   // sum of the segments after i
      acc += x;
    }
  }
  __syncthreads();
  float acc = tot[tid];
  float* dst = dlg + (size_t)row * L;
  for (int j = hi - 1; j >= lo; --j) {
    acc += value(j);
    dst[j] = acc;
  }
}

// ----------------------------------------------------------------------------
// host launchers
// ----------------------------------------------------------------------------
int gla_padded_dim(int n);

template <int FP, int DP, typename OutT>
static hipError_t launch_gla_bwd_t(const void* fq, const void* fk, const void* v, const float* lg,
                                   const void* dy, void* dfq, void* dfk, void* dv, float* dlg,
                                   int B, int H, int L, int F, int D, int gate_per_head, float* ws,
                                   hipStream_t st) {
  const size_t BHL = (size_t)B * H * L;
  float* den = ws;
  float* delta = den + BHL;
  float* p = delta + BHL;
  float* dG = p + BHL;
  auto ka = gla_bwd_a_kernel<FP, DP, OutT>;
  auto kb = gla_bwd_b_kernel<FP, DP, OutT>;
  constexpr int lds_a = BwdACfg<FP, DP>::BYTES, lds_b = BwdBCfg<FP, DP>::BYTES;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(ka),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, lds_a);
  if (e != hipSuccess) return e;
  e = hipFuncSetAttribute(reinterpret_cast<const void*>(kb),
                          hipFuncAttributeMaxDynamicSharedMemorySize, lds_b);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(ka, dim3(B * H), dim3(256), lds_a, st, (const bf16*)fq,
                     (const bf16*)fk, (const bf16*)v, lg, (const bf16*)dy, (OutT*)dfq, den, delta,
                     p, H, L, F, D, gate_per_head);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(kb, dim3(B * H), dim3(256), lds_b, st, (const bf16*)fq,
                     (const bf16*)fk, (const bf16*)v, lg, (const bf16*)dy, den, delta, p,
                     (OutT*)dfk, (OutT*)dv, dG, H, L, F, D, gate_per_head);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  hipLaunchKernelGGL(gla_gate_grad_kernel, dim3(gate_per_head ? B * H : B), dim3(256), 0, st, dG,
                     dlg, H, L, gate_per_head);
  return hipGetLastError();
}

size_t gla_bwd_workspace(int B, int H, int L) { return (size_t)4 * B * H * L * sizeof(float); }

hipError_t launch_gla_bwd(const void* fq, const void* fk, const void* v, const float* lg,
                          const void* dy, void* dfq, void* dfk, void* dv, float* dlg,
                          bool grad_bf16, int B, int H, int L, int F, int D, int gate_per_head,
                          float* ws, hipStream_t st) {
  const int fp = gla_padded_dim(F), dp = gla_padded_dim(D);
#define LZ_GLA_BWD(FPV, DPV)                                                                   \
  if (fp == FPV && dp == DPV)                                                                  \
    return grad_bf16 ? launch_gla_bwd_t<FPV, DPV, bf16>(fq, fk, v, lg, dy, dfq, dfk, dv, dlg,  \
                                                         B, H, L, F, D, gate_per_head, ws, st) \
                     : launch_gla_bwd_t<FPV, DPV, float>(fq, fk, v, lg, dy, dfq, dfk, dv, dlg, \
                                                          B, H, L, F, D, gate_per_head, ws, st);
  LZ_GLA_BWD(32, 32) LZ_GLA_BWD(32, 64) LZ_GLA_BWD(32, 128)
  LZ_GLA_BWD(64, 32) LZ_GLA_BWD(64, 64) LZ_GLA_BWD(64, 128)
  LZ_GLA_BWD(128, 32) LZ_GLA_BWD(128, 64) LZ_GLA_BWD(128, 128)
  LZ_GLA_BWD(256, 32) LZ_GLA_BWD(256, 64)
#undef LZ_GLA_BWD
  return hipErrorInvalidValue;
}

}  // namespace lz
