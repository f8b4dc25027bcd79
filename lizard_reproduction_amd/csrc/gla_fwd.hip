// Chunked gated linear attention, forward, for gfx950.
//
// Math (reference operator src/kernels/gla.py:259-263 with the chunk
// conventions of src/kernels/gla.py:19-101; dense form
// src/lizard_attention.py:20-31).  Per (b, h), tokens are cut into 64-token
// chunks.  Inside chunk n, lg_j is the inclusive sum of log_gamma over the
// chunk up to token j (so every absorbed factor exp(.) is <= 1):
//   Q~_i = bf16(fq_i e^{lg_i}),  K~_t = bf16(fk_t e^{lg_end - lg_t})
//   a_it = bf16((fq_i . fk_t) e^{lg_i - lg_t}) for t <= i
//   o_i  = Q~_i S_n + sum_t a_it v_t,  den_i = Q~_i . z_n + sum_t a_it
//   y_i  = o_i / max(den_i, FLT_MIN)
//   S_{n+1} = e^{lg_end} S_n + K~^T V,   z_{n+1} = e^{lg_end} z_n + sum_t K~_t
// The reference takes the same differences from a global cumsum G; the
// chunk-local sums here are the same numbers without the cancellation.
//
// One workgroup (4 waves) per (b, h) walks the chunks in order.  The state
// S (F x D, fp32) lives in MFMA accumulator registers for the whole walk and
// is never written to HBM: HBM traffic is one read of fq, fk, v and the gate,
// and one write of y.  Per chunk:
//   1. stage fq, fk (natural, [token][f]) and fk, v (transposed, [f|d][token])
//      in LDS; wave 0 scans the gate.
//   2. each wave computes one 32x32 tile of s^T = fk fq^T (keys x queries),
//      applies the causal decay in registers, rounds to bf16 and publishes
//      the tile to LDS as ready-made MFMA B operands; partial row sums and
//      Q~.z partials go to LDS.
//   3. each wave forms o^T = S^T Q~^T + V^T P^T for its d-tile (S operands
//      come straight from its accumulators), divides by den and stores y;
//      then S <- e^{lg_end} S + K~^T V for its d-tile and z is updated.
// Inputs: fq, fk [BH, L, F] bf16; v [BH, L, D] bf16; log_gamma fp32
// [B, L] (gate_heads == 1) or [B, H, L] (gate_heads == H).  Output y bf16.
#include "common.hpp"

namespace lz {

template <int FP, int DP>
struct GlaFwdCfg {
  static constexpr int C = 64;
  static constexpr int NPITCH = FP + 8;   // natural tiles [64][NPITCH]
  static constexpr int TPITCH = C + 8;    // transposed tiles [FP|DP][TPITCH]
  static constexpr int NFT = FP / 32, NDT = DP / 32;
  static constexpr int DT_PER_WAVE = NDT >= 4 ? NDT / 4 : 1;
  static constexpr int QT_PER_WAVE = NDT >= 4 ? 2 : 1;
  // LDS carve-up (bytes)
  static constexpr int OFF_FQN = 0;
  static constexpr int OFF_FKN = OFF_FQN + C * NPITCH * 2;
  static constexpr int OFF_FKT = OFF_FKN + C * NPITCH * 2;
  static constexpr int OFF_VT = OFF_FKT + FP * TPITCH * 2;
  static constexpr int OFF_PF = OFF_VT + DP * TPITCH * 2;          // [2 qt][4 kb][64][8] bf16
  static constexpr int OFF_RS = OFF_PF + 2 * 4 * 64 * 16;          // [2][64] f32
  static constexpr int OFF_QZ = OFF_RS + 2 * 64 * 4;               // [4][64] f32
  static constexpr int OFF_LG = OFF_QZ + 4 * 64 * 4;               // [64] f32 chunk-local scan
  static constexpr int OFF_QS = OFF_LG + 64 * 4;                   // [64] e^{lg}
  static constexpr int OFF_KS = OFF_QS + 64 * 4;                   // [64] e^{end-lg}, slot order
  static constexpr int OFF_Z = OFF_KS + 64 * 4;                    // [FP] z, slot order
  static constexpr int OFF_R = OFF_Z + FP * 4;                     // chunk decay
  static constexpr int BYTES = OFF_R + 16;
};

template <int FP, int DP>
__global__ __launch_bounds__(256) void gla_fwd_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, bf16* __restrict__ y, int H, int L, int F, int D,
    int gate_per_head) {
  using Cfg = GlaFwdCfg<FP, DP>;
  constexpr int C = Cfg::C, NP = Cfg::NPITCH, TP = Cfg::TPITCH;
  constexpr int NFT = Cfg::NFT, NDT = Cfg::NDT;
  extern __shared__ __align__(16) char smem[];
  bf16* fqn = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQN);
  bf16* fkn = reinterpret_cast<bf16*>(smem + Cfg::OFF_FKN);
  bf16* fkt = reinterpret_cast<bf16*>(smem + Cfg::OFF_FKT);
  bf16* vt = reinterpret_cast<bf16*>(smem + Cfg::OFF_VT);
  bf16x8* pf = reinterpret_cast<bf16x8*>(smem + Cfg::OFF_PF);
  float* rs = reinterpret_cast<float*>(smem + Cfg::OFF_RS);
  float* qz = reinterpret_cast<float*>(smem + Cfg::OFF_QZ);
  float* lgs = reinterpret_cast<float*>(smem + Cfg::OFF_LG);
  float* qs = reinterpret_cast<float*>(smem + Cfg::OFF_QS);
  float* kss = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  float* zs = reinterpret_cast<float*>(smem + Cfg::OFF_Z);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  const int bh = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const bf16* fqb = fq + (size_t)bh * L * F;
  const bf16* fkb = fk + (size_t)bh * L * F;
  const bf16* vb = v + (size_t)bh * L * D;
  bf16* yb = y + (size_t)bh * L * D;
  const float* lgb = log_gamma + (size_t)(gate_per_head ? bh : bh / H) * L;

  for (int f = tid; f < FP; f += 256) zs[f] = 0.f;

  // wave -> (d-tiles, q-tiles) of the output; S tiles follow the d-tiles
  const bool active = NDT >= 2 || wave < 2;
  f32x16 S[Cfg::DT_PER_WAVE][NFT];
#pragma unroll
  for (int i = 0; i < Cfg::DT_PER_WAVE; ++i)
#pragma unroll
    for (int ft = 0; ft < NFT; ++ft) S[i][ft] = zero16();

  const int NT = (L + C - 1) / C;
  for (int n = 0; n < NT; ++n) {
    const int t0 = n * C;
    __syncthreads();
    // ---- 1. stage the chunk -------------------------------------------------
    {
      constexpr int F4 = FP / 4;
      for (int idx = tid; idx < C * F4; idx += 256) {
        const int r = idx / F4, c = (idx % F4) * 4;
        const bf16x4 a = load4(fqb, t0 + r, c, L, F);
        const bf16x4 b = load4(fkb, t0 + r, c, L, F);
        *reinterpret_cast<bf16x4*>(fqn + r * NP + pidx(c)) = a;
        *reinterpret_cast<bf16x4*>(fkn + r * NP + pidx(c)) = b;
#pragma unroll
        for (int e = 0; e < 4; ++e) fkt[(c + e) * TP + pidx(r)] = b[e];
      }
      constexpr int D4 = DP / 4;
      for (int idx = tid; idx < C * D4; idx += 256) {
        const int r = idx / D4, c = (idx % D4) * 4;
        const bf16x4 b = load4(vb, t0 + r, c, L, D);
#pragma unroll
        for (int e = 0; e < 4; ++e) vt[(c + e) * TP + pidx(r)] = b[e];
      }
      if (wave == 0) {
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
    }
    __syncthreads();
    // ---- 2. scores, P fragments, row sums, Q~.z partials ---------------------
    {
      const int kt = wave >> 1, qt = wave & 1;
      f32x16 s = zero16();
#pragma unroll
      for (int kb = 0; kb < FP / 16; ++kb) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(fkn + (kt * 32 + col) * NP + 16 * kb + 8 * h);
        const bf16x8 b = *reinterpret_cast<const bf16x8*>(fqn + (qt * 32 + col) * NP + 16 * kb + 8 * h);
        s = mfma(a, b, s);
      }
      const int qi = qt * 32 + col;
      const float lgq = lgs[qi];
      bf16x8 p[2];
      float rsum = 0.f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kt * 32 + acc_row(r, h);
        const float val = key <= qi ? s[r] * fexp(lgq - lgs[key]) : 0.f;
        const bf16 pb = to_bf16(val);
        p[r >> 3][r & 7] = pb;
        rsum += to_f32(pb);
      }
      rsum += xhalf(rsum);
      pf[(qt * 4 + kt * 2 + 0) * 64 + lane] = p[0];
      pf[(qt * 4 + kt * 2 + 1) * 64 + lane] = p[1];
      if (h == 0) rs[kt * 64 + qi] = rsum;
      // Q~ . z partial over a quarter of the features; query = lane
      constexpr int FQ = FP / 4;
      const float qsv = qs[lane];
      float acc = 0.f;
      for (int f = wave * FQ; f < (wave + 1) * FQ; ++f)
        acc += to_f32(to_bf16(to_f32(fqn[lane * NP + f]) * qsv)) * zs[f];
      qz[wave * 64 + lane] = acc;
    }
    __syncthreads();
    // ---- 3. outputs and state update ----------------------------------------
    const float r_n = rdec[0];
    if (active) {
#pragma unroll
      for (int i = 0; i < Cfg::DT_PER_WAVE; ++i) {
        const int dt = NDT >= 4 ? wave + 4 * i : (NDT == 2 ? (wave >> 1) : 0);
        bf16x8 sa[FP / 16];
#pragma unroll
        for (int kb = 0; kb < FP / 16; ++kb) sa[kb] = acc_operand(S[i][kb >> 1], kb & 1);
#pragma unroll
        for (int j = 0; j < Cfg::QT_PER_WAVE; ++j) {
          const int qt = NDT >= 4 ? j : (wave & 1);
          const int qi = qt * 32 + col;
          const float qsv = qs[qi];
          f32x16 o = zero16();
#pragma unroll
          for (int kb = 0; kb < FP / 16; ++kb) {
            const bf16x8 raw = *reinterpret_cast<const bf16x8*>(fqn + qi * NP + 16 * kb + 8 * h);
            bf16x8 b;
#pragma unroll
            for (int e = 0; e < 8; ++e) b[e] = to_bf16(to_f32(raw[e]) * qsv);
            o = mfma(sa[kb], b, o);
          }
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(vt + (dt * 32 + col) * TP + 16 * kb + 8 * h);
            o = mfma(a, pf[(qt * 4 + kb) * 64 + lane], o);
          }
          const float den = rs[qi] + rs[64 + qi] + qz[qi] + qz[64 + qi] + qz[128 + qi] + qz[192 + qi];
          const float inv = 1.f / fmaxf(den, TINY);
          const int tok = t0 + qi;
          if (tok < L) {
#pragma unroll
            for (int g = 0; g < 4; ++g)
              store4<bf16>(yb, tok, dt * 32 + 8 * g + 4 * h, D, o[4 * g] * inv,
                           o[4 * g + 1] * inv, o[4 * g + 2] * inv, o[4 * g + 3] * inv);
          }
        }
        // S <- e^{lg_end} S + K~^T V  (this wave's d-tile)
#pragma unroll
        for (int ft = 0; ft < NFT; ++ft) {
#pragma unroll
          for (int r = 0; r < 16; ++r) S[i][ft][r] *= r_n;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) {
            const bf16x8 raw = *reinterpret_cast<const bf16x8*>(fkt + (ft * 32 + col) * TP + 16 * kb + 8 * h);
            bf16x8 a;
#pragma unroll
            for (int e = 0; e < 8; ++e) a[e] = to_bf16(to_f32(raw[e]) * kss[16 * kb + 8 * h + e]);
            const bf16x8 b = *reinterpret_cast<const bf16x8*>(vt + (dt * 32 + col) * TP + 16 * kb + 8 * h);
            S[i][ft] = mfma(a, b, S[i][ft]);
          }
        }
      }
    }
    // z <- e^{lg_end} z + sum_t K~_t   (zs in slot order of f)
    for (int fs = tid; fs < FP; fs += 256) {
      const int f = pidx(fs);
      float acc = 0.f;
      for (int t = 0; t < C; ++t) acc += to_f32(to_bf16(to_f32(fkt[f * TP + t]) * kss[t]));
      zs[fs] = zs[fs] * r_n + acc;
    }
  }
}

template <int FP, int DP>
static hipError_t launch_gla_fwd_t(const void* fq, const void* fk, const void* v,
                                   const float* lg, void* y, int B, int H, int L, int F, int D,
                                   int gate_per_head, hipStream_t st) {
  using Cfg = GlaFwdCfg<FP, DP>;
  auto kern = gla_fwd_kernel<FP, DP>;
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, Cfg::BYTES);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(kern, dim3(B * H), dim3(256), Cfg::BYTES, st, (const bf16*)fq,
                     (const bf16*)fk, (const bf16*)v, lg, (bf16*)y, H, L, F, D, gate_per_head);
  return hipGetLastError();
}

int gla_padded_dim(int n) {
  if (n <= 32) return 32;
  if (n <= 64) return 64;
  if (n <= 128) return 128;
  if (n <= 256) return 256;
  return -1;
}

hipError_t launch_gla_fwd(const void* fq, const void* fk, const void* v, const float* lg, void* y,
                          int B, int H, int L, int F, int D, int gate_per_head, hipStream_t st) {
  const int fp = gla_padded_dim(F), dp = gla_padded_dim(D);
#define LZ_GLA_FWD(FPV, DPV) \
  if (fp == FPV && dp == DPV) \
    return launch_gla_fwd_t<FPV, DPV>(fq, fk, v, lg, y, B, H, L, F, D, gate_per_head, st);
  LZ_GLA_FWD(32, 32) LZ_GLA_FWD(32, 64) LZ_GLA_FWD(32, 128)
  LZ_GLA_FWD(64, 32) LZ_GLA_FWD(64, 64) LZ_GLA_FWD(64, 128)
  LZ_GLA_FWD(128, 32) LZ_GLA_FWD(128, 64) LZ_GLA_FWD(128, 128)
  LZ_GLA_FWD(256, 32) LZ_GLA_FWD(256, 64)
#undef LZ_GLA_FWD
  return hipErrorInvalidValue;
}

bool gla_dims_supported(int F, int D) {
  const int fp = gla_padded_dim(F), dp = gla_padded_dim(D);
  if (fp < 0 || dp < 0) return false;
  return dp <= 128 && (fp <= 128 || dp <= 64);
}

}  // namespace lz
