// Chunked gated linear attention, backward, for gfx950.
//
// Reference: _GLA.backward and its kernels (src/kernels/gla.py:104-194,
// 236-256), with the autograd steps of the gate path (gla.py:260-262).  With
// the chunk-local notation of gla_fwd.hip (lg, qs = e^{lg}, ks = e^{lg_end-lg},
// r = e^{lg_end}, decay_it = e^{lg_i - lg_t}), S_n, z_n the forward state
// entering chunk n, and dS, dz the gradient state flowing back into chunk n
// from the chunks after it:
//   delta_i = dy_i . y_i                              (fp32 y)
//   dA_it   = [t<=i] (dy_i . v_t - delta_i) / den_i,  dad = dA * decay
//   dfq_i   = sum_t dad_it fk_t + (qs_i/den_i) (dy_i S_n^T - delta_i z_n)
//   dfk_t   = sum_i dad_it fq_i + ks_t (v_t dS^T - dz)
//   dv_t    = sum_i (a_it/den_i) dy_i + ks_t (fk_t dS)
//   dS <- r_n dS + Q^_n^T dy_n,  Q^_i = bf16(fq_i qs_i / den_i)   (after chunk n)
//   dz <- r_n dz + sum_i fq_i (qs_i delta_i / den_i)
//   dG_j    = fq_j . dfq_j - fk_j . dfk_j,  d log_gamma = reverse cumsum of dG
//             (summed over heads for a per-token gate)
//
// Launches (G = segments per (b, h), as in the forward; no state goes to HBM
// except the per-segment records when G > 1):
//   [G > 1] forward segment pass + scan (gla_fwd.hip): S, z entering each segment
//   A  gla_bwd_dq_kernel, forward walk per (b, h, segment): carries S^T in
//      MFMA accumulators; recomputes den and delta -- delta_i = dy_i . o_i /
//      den_i with dy_i . o_i = Q~_i . (S_n dy_i) + sum_t a_it (v_t . dy_i), both
//      products it needs anyway, Q~ = fq qs unrounded as in the forward -- and
//      writes dfq, den, delta and fq . dfq.
//   [G > 1] gla_bwd_state_kernel + reverse scan: dS, dz entering each segment
//      from the right (needs den and delta from A).
//   B  gla_bwd_dkv_kernel, reverse walk per (b, h, segment): carries dS in
//      accumulators and publishes it as bf16 dS^T in LDS each chunk (dv
//      contracts the state over f straight from the accumulators, dfk over d
//      through LDS transpose reads); writes dv, dfk and dG.
//   gate: d log_gamma = reverse cumsum of dG over L (head-summed for a
//      per-token gate), one launch (gla_gate_grad_kernel) from dG and the
//      per-chunk dG totals kernel B writes; with a per-head gate and G = 1
//      kernel B, whose reverse walk sees the whole row, writes it instead.
//   With G = 1, A and B of a (b, h) run in one workgroup, B right after A
//   (gla_bwd_fused_kernel): B then needs only that workgroup's den, delta and
//   p, and starts on the chunks A read last.
// Operand staging follows gla_fwd.hip: row-major tiles in LDS, operands that
// contract over tokens from LDS transpose reads, next chunk prefetched into
// registers.
#include "gla_common.hpp"

namespace lz {

template <int FP, int DP>
struct BwdCommon {
  static constexpr int C = GLA_C;
  static constexpr int PF = lds_pitch(FP), PD = lds_pitch(DP);
  static constexpr int NFT = FP / 32, NDT = DP / 32;
  static constexpr int NLF = C * FP / 8 / 256, NLD = C * DP / 8 / 256;
  static constexpr int SEG = SegRec<FP, DP>::SIZE;
};

// ============================================================================
// Both walks run eight waves (512 threads) per workgroup: a chunk's LDS
// leaves room for one workgroup per CU, so the second wave per SIMD comes
// from inside it.  Chunk tiles are loaded and stored by all 512 threads.
// ============================================================================
constexpr int B_WAVES = 8;
constexpr int B_THREADS = 64 * B_WAVES;

// Rows [t0, t0+64) of a [L x ncols] bf16 matrix into registers by B_THREADS
// threads (item idx = tid + B_THREADS i: row idx / (KP/8), 8 columns), zero
// outside the matrix; items past the tile are skipped.
template <int KP, int N>
__device__ __forceinline__ void load_tile8(uint4 (&reg)[N], const bf16* __restrict__ base, int t0,
                                           int L, int ncols, bool vec) {
  load_items<KP, B_THREADS, N, GLA_C * KP / 8>(reg, base, t0, L, ncols, vec);
}

template <int KP, int N>
__device__ __forceinline__ void store_tile8(const uint4 (&reg)[N], bf16* tile, int pitch) {
  constexpr int K8 = KP / 8, ITEMS = GLA_C * K8;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int idx = threadIdx.x + B_THREADS * i;
    if (ITEMS % B_THREADS == 0 || idx < ITEMS)
      *reinterpret_cast<uint4*>(tile + (idx / K8) * pitch + (idx % K8) * 8) = reg[i];
  }
}

// ============================================================================
// kernel A: forward walk -> dfq, den, delta, p = fq . dfq
//
//   phase 1  waves 0-3: the score tile (keys kt x queries qt) a^T and v dy^T,
//            the decay, sum_t a and sum_t a (v . dy) (the tile of keys 32-63 x
//            queries 0-31 is causally zero: its wave forms half of Q~ . z
//            instead); waves 4-7: the other half of Q~ . z, K~ = bf16(fk ks)
//            with its column sums; X jobs (f-tile, query half): X = S dy^T
//            and qs fq . X, waves 4-7 first;
//   phase 2  waves 0-3: den, delta, dad fragments; waves 4-7: the z update;
//   phase 3  X jobs: dfq and fq . dfq; S^T tiles: S^T <- r S^T + V^T K~;
//   tail     p, next chunk, publish S.
// S lives in the accumulators of the waves that own its tiles.  With FP = 256
// (eight f-tiles) wave w owns f-tile w across all d-tiles and contracts its X
// jobs from its own registers; otherwise tile t = wave + 8 i is owned
// (f-tile t % NFT, d-tile t / NFT) and the tiles are published as bf16 S
// [f][d] in LDS each chunk, where the X jobs read them.
// ============================================================================
template <int FP, int DP>
struct BwdA : BwdCommon<FP, DP> {
  using B_ = BwdCommon<FP, DP>;
  static constexpr int C = B_::C, PF = B_::PF, PD = B_::PD, NFT = B_::NFT, NDT = B_::NDT;
  static constexpr bool SREG = NFT >= B_WAVES;    // S by f-tile in registers, no LDS copy
  static constexpr int S_OWN = SREG ? NDT * (NFT / B_WAVES) : (NFT * NDT + B_WAVES - 1) / B_WAVES;
  static constexpr int XJ = SREG ? 2 * (NFT / B_WAVES) : 1;   // X jobs per wave
  // chunks in flight while one computes (a second register set measured
  // slower at the bench shapes, and spills at the largest tiles)
  static constexpr int DEPTH = 1;
  static constexpr int NLF = (C * FP / 8 + B_THREADS - 1) / B_THREADS;
  static constexpr int NLD = (C * DP / 8 + B_THREADS - 1) / B_THREADS;
  static constexpr int OFF_FQ = 0;
  static constexpr int OFF_FK = OFF_FQ + C * PF * 2;
  static constexpr int OFF_V = OFF_FK + C * PF * 2;
  static constexpr int OFF_DY = OFF_V + C * PD * 2;
  static constexpr int OFF_KT = OFF_DY + C * PD * 2;       // K~ = bf16(fk ks), row-major
  static constexpr int OFF_SL = OFF_KT + C * PF * 2;       // S [f][d] bf16 (not SREG)
  static constexpr int OFF_FR = OFF_SL + (SREG ? 0 : FP * PD * 2);   // dad fragments
  static constexpr int OFF_RA = OFF_FR + 2 * 4 * 64 * 16;  // [2][64] sum_t a
  static constexpr int OFF_RAV = OFF_RA + 2 * 64 * 4;      // [2][64] sum_t a (v . dy)
  static constexpr int OFF_QZ = OFF_RAV + 2 * 64 * 4;      // [6][64] Q~ . z partials
  static constexpr int OFF_NX = OFF_QZ + 6 * 64 * 4;       // [NFT][64] Q~ . (S dy) partials
  static constexpr int OFF_PP = OFF_NX + NFT * 64 * 4;     // [NFT][64] fq . dfq partials
  static constexpr int OFF_DEN = OFF_PP + NFT * 64 * 4;
  static constexpr int OFF_DEL = OFF_DEN + 64 * 4;
  static constexpr int OFF_LG = OFF_DEL + 64 * 4;
  static constexpr int OFF_QS = OFF_LG + 64 * 4;
  static constexpr int OFF_KS = OFF_QS + 64 * 4;
  static constexpr int OFF_Z = OFF_KS + 64 * 4;
  static constexpr int OFF_ZP = OFF_Z + 2 * FP * 4;        // 2048 partial sums of K~
  static constexpr int OFF_R = OFF_ZP + 2048 * 4;
  static constexpr int BYTES = OFF_R + 16;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
};

// qz[lane] = qs_lane (fq_lane . z) over features [f0, f0 + NF) (query = lane)
template <int NF>
__device__ __forceinline__ void qz_part(const bf16* fq_l, int pitch, const float* zs,
                                        const float* qs, float* qz, int lane, int f0) {
  float acc = 0.f;
#pragma unroll
  for (int c = 0; c < NF; c += 8) {
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(fq_l + lane * pitch + f0 + c);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc += to_f32(x[e]) * zs[f0 + c + e];
  }
  qz[lane] = acc * qs[lane];
}

// z_next = r z + (column sums of K~) by 256 threads t: 256 / KP adjacent
// threads per feature, each adding eight of scale_rows' partial sums, then
// combined by lane exchanges
template <int KP>
__device__ __forceinline__ void z_update(float* zn, const float* zs, const float* part, float r,
                                         int t) {
  constexpr int TPF = 256 / KP, PER = RowItems<KP>::PARTS / TPF;
  static_assert(PER == 8, "eight partial sums per thread");
  const int f = t / TPF, sub = t % TPF;
  float s = 0.f;
#pragma unroll
  for (int p = 0; p < PER; ++p) s += part[(sub * PER + p) * KP + f];
#pragma unroll
  for (int off = 1; off < TPF; off <<= 1) s += __shfl_xor(s, off);
  if (sub == 0) zn[f] = zs[f] * r + s;
}

// EXT (one F tile of a split feature dimension): den and delta are not
// formed from this tile's features but read from den_out / delta_out, where
// the caller has put those of the whole feature dimension; the kernel then
// writes this tile's share of every gradient.
template <int FP, int DP, typename OutT, bool VEC, bool EXT, bool FOLD = false>
__device__ __forceinline__ void gla_bwd_dq_body(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, const bf16* __restrict__ dy, OutT* __restrict__ dfq,
    float* __restrict__ den_out, float* __restrict__ delta_out, float* __restrict__ p_out,
    const float* __restrict__ seg_state, int H, int L, int F, int D, int gate, int G,
    int cps, int M, int KG, int xper, int nxcd, int nblk, const float* __restrict__ seg_lam) {
  using Cfg = BwdA<FP, DP>;
  constexpr int C = Cfg::C, PF = Cfg::PF, PD = Cfg::PD;
  constexpr int NFT = Cfg::NFT, NDT = Cfg::NDT;
  // LDS operands are read PIPE products ahead of their MFMAs (one at F = 256,
  // where two would spill)
  constexpr int PIPE = FP >= 256 ? 1 : 2;
  constexpr bool SREG = Cfg::SREG;
  extern __shared__ __align__(16) char smem[];
  bf16* fq_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQ);
  bf16* fk_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FK);
  bf16* v_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_V);
  bf16* dy_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_DY);
  bf16* kt_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_KT);
  bf16* s_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_SL);
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
  float* ks = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  // z entering chunk n in zb + FP (n & 1): the update for chunk n + 1 is
  // written while phase 3 still reads chunk n's
  float* zb = reinterpret_cast<float*>(smem + Cfg::OFF_Z);
  float* zp = reinterpret_cast<float*>(smem + Cfg::OFF_ZP);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  // a workgroup walks M consecutive segments (seg .. seg + M - 1)
  const int nwg = G / M;
  int blk;
  if (!walk_block(xper, nxcd, nblk, blk)) return;
  const int bh = blk / nwg, seg = (blk % nwg) * M;
  const int n0 = seg * cps, n1 = min((L + C - 1) / C, n0 + M * cps);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const bool vecF = VEC || (F & 7) == 0, vecD = VEC || (D & 7) == 0;
  const size_t offF = (size_t)bh * L * F, offD = (size_t)bh * L * D, offL = (size_t)bh * L;
  // fk and v of the kv head of this query head (KG query heads share one)
  const size_t offFk = (size_t)(bh / KG) * L * F, offDv = (size_t)(bh / KG) * L * D;
  const float* lgb = log_gamma + (size_t)((gate & GATE_PER_HEAD) ? bh : bh / H) * L;
  // the forward state entering segment seg: its scanned record, or (FOLD) the
  // local records of segments 0 .. seg - 1 folded here (their total log
  // decays at seg_lam)
  const int own = seg_owner_uniform(bh, KG, gate);
  const float* st =
      G > 1 ? seg_state + ((size_t)own * G + (FOLD ? 0 : seg)) * Cfg::SEG : nullptr;

  // owned S^T tiles (rows d, columns f): i -> (f-tile, d-tile)
  auto s_tile = [&](int i, int& ft, int& dt) __attribute__((always_inline)) -> bool {
    if constexpr (SREG) {
      ft = wave * (NFT / B_WAVES) + i / NDT;
      dt = i % NDT;
      return true;
    } else {
      const int t = wave + B_WAVES * i;
      ft = t % NFT;
      dt = t / NFT;
      return t < NFT * NDT;
    }
  };
  // X jobs of this wave: j -> (f-tile, query half)
  auto x_job = [&](int j, int& ft, int& hq) __attribute__((always_inline)) -> bool {
    if constexpr (SREG) {
      ft = wave * (NFT / B_WAVES) + (j >> 1);
      hq = j & 1;
      return true;
    } else {
      // waves 4-7 take jobs 0-3; the two waves of a SIMD (w, w + 4) take
      // opposite query halves, whose phase-3 products differ in number
      const int job = ((wave + 4) & 7) ^ (wave >> 2);
      ft = job >> 1;
      hq = job & 1;
      return job < 2 * NFT;
    }
  };
  f32x16 St[Cfg::S_OWN];
  if constexpr (FOLD) {   // folded in LDS, before the first chunk is staged there
    static_assert(Cfg::SEG * 4 <= Cfg::BYTES, "a folded record fits the chunk's LDS");
    float* fold_l = reinterpret_cast<float*>(smem);
    if (seg > 0)
      fold_records<B_THREADS, Cfg::SEG, 160>(fold_l, st, seg_lam + (size_t)own * G, 0, 1, seg);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < Cfg::S_OWN; ++i) {
      St[i] = zero16();
      int ft, dt;
      if (s_tile(i, ft, dt) && seg > 0) {
        const int f = ft * 32 + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) St[i][r] = fold_l[f * DP + dt * 32 + acc_row(r, h)];
      }
    }
    static_assert(FP <= B_THREADS, "one z element per thread");
    const float zv = seg > 0 && tid < FP ? fold_l[FP * DP + tid] : 0.f;
    __syncthreads();   // read before the LDS is reused
    if (tid < FP) zb[FP * (n0 & 1) + tid] = zv;
  } else {
#pragma unroll
    for (int i = 0; i < Cfg::S_OWN; ++i) {
      St[i] = zero16();
      int ft, dt;
      if (s_tile(i, ft, dt) && st) {
        const int f = ft * 32 + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) St[i][r] = st[f * DP + dt * 32 + acc_row(r, h)];
      }
    }
    for (int f = tid; f < FP; f += B_THREADS) zb[FP * (n0 & 1) + f] = st ? st[FP * DP + f] : 0.f;
  }
  // bf16 S [f][d] for the X jobs (4 consecutive d per store)
  auto publish = [&]() __attribute__((always_inline)) {
    if constexpr (!SREG) {
#pragma unroll
      for (int i = 0; i < Cfg::S_OWN; ++i) {
        int ft, dt;
        if (s_tile(i, ft, dt)) {
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            bf16x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = to_bf16(St[i][4 * g4 + e]);
            *reinterpret_cast<bf16x4*>(s_l + (ft * 32 + col) * PD + dt * 32 + 8 * g4 + 4 * h) = o;
          }
        }
      }
    }
  };

  // per-chunk single-wave work goes to waves whose tail is otherwise light:
  // the gate to wave 3, fq . dfq to wave 2 (the z update runs in phase 2, on
  // waves 4-7)
  constexpr int GW = 3, PW = 2;
  // DEPTH register sets: while chunk n computes, chunks n+1 .. n+DEPTH are in flight
  constexpr int DEPTH = Cfg::DEPTH;
  uint4 rq[DEPTH][Cfg::NLF], rk[DEPTH][Cfg::NLF], rv[DEPTH][Cfg::NLD], rd[DEPTH][Cfg::NLD];
  float rg[DEPTH] = {};
  bool rgok[DEPTH] = {};
  auto issue = [&](auto set, int n) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    if (n < n1) {
      load_tile8<FP>(rq[S], fq + offF, n * C, L, F, vecF);
      load_tile8<FP>(rk[S], fk + offFk, n * C, L, F, vecF);
      load_tile8<DP>(rv[S], v + offDv, n * C, L, D, vecD);
      load_tile8<DP>(rd[S], dy + offD, n * C, L, D, vecD);
      if (wave == GW) {
        rg[S] = gate_at(lgb, n * C + lane, L);
        rgok[S] = n * C + lane < L;
      }
    }
  };
  auto stage = [&](auto set) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    store_tile8<FP>(rq[S], fq_l, PF);
    store_tile8<FP>(rk[S], fk_l, PF);
    store_tile8<DP>(rv[S], v_l, PD);
    store_tile8<DP>(rd[S], dy_l, PD);
    if (wave == GW) gate_scan(rg[S], lane, lgs, qs, ks, rdec, gate, rgok[S]);
  };
  issue(SET0, n0);
  if constexpr (DEPTH == 2) issue(SET1, n0 + 1);
  stage(SET0);
  publish();
  __syncthreads();

  const bool scorer = wave < 4;
  const int kt = (wave >> 1) & 1, qt = wave & 1;   // score tile of waves 0-3
  const int qi = qt * 32 + col;                     // its query (lane)
  // keys 32-63 x queries 0-31 (wave 2) is causally zero: its row sums are 0,
  // its dad fragments are never read (phase 3 skips them)
  const bool live = scorer && !(kt == 1 && qt == 0);
  // chunk n is in LDS and register set `set` is free; the next set holds chunk n+1
  auto step = [&](auto set, int n) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    const int t0 = n * C;
    const float* zs = zb + FP * (n & 1);
    // waves 0-3 load the next chunk now, waves 4-7 once their phase-1 work is
    // done: issued together, the later waves' loads waited for free slots in
    // the CU's memory queue and held back their phase-1 work
    if (wave < 4) issue(set, n + DEPTH);
    // ---- phase 1 ---------------------------------------------------------------
    f32x16 vdy = zero16();
    float dec[16];   // causal decay of the score tile, reused in phase 2
    if (scorer && !live) {
      if (h == 0) {
        ra[kt * 64 + qi] = 0.f;
        rav[kt * 64 + qi] = 0.f;
      }
      // qs (fq . z) over the first two quarters of the features (all four
      // at FP = 256, where two more partial sums in den made the kernel spill
      // registers); query = lane
#pragma unroll
      for (int q4 = 0; q4 < (FP >= 256 ? 4 : 2); ++q4)
        qz_part<FP / 4>(fq_l, PF, zs, qs, qz + 64 * q4, lane, q4 * (FP / 4));
    } else if (scorer) {
      f32x16 aT = mfma_chain<FP / 16, PIPE>(
          zero16(), [&](int kb) { return row_operand(fk_l, PF, kt * 32 + col, 16 * kb, h); },
          [&](int kb) { return row_operand(fq_l, PF, qi, 16 * kb, h); });
      vdy = mfma_chain<DP / 16, PIPE>(
          vdy, [&](int kb) { return row_operand(v_l, PD, kt * 32 + col, 16 * kb, h); },
          [&](int kb) { return row_operand(dy_l, PD, qi, 16 * kb, h); });
      const float lgq = lgs[qi];
      float sa = 0.f, sav = 0.f;
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        const int k0 = kt * 32 + 8 * g4 + 4 * h;   // keys of registers 4 g4 .. +4
        const f32x4 lk = *reinterpret_cast<const f32x4*>(lgs + k0);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * g4 + e;
          dec[r] = k0 + e <= qi ? fexp(lgq - lk[e]) : 0.f;
          aT[r] = to_f32(to_bf16(aT[r] * dec[r]));   // a exactly as the forward rounds it
          sa += aT[r];
          sav += aT[r] * vdy[r];
        }
      }
      sa += xhalf(sa);
      sav += xhalf(sav);
      if (h == 0) {
        ra[kt * 64 + qi] = sa;
        rav[kt * 64 + qi] = sav;
      }
    } else {
      // K~ = bf16(fk ks) once per chunk (the forward's rounding), with its
      // column sums for z
      {
        uint4 kti[RowItems<FP>::N];
        scale_rows_t<FP>(fk_l, PF, ks, kti, zp, tid - 256);
        store_rows_t<FP>(kti, kt_l, PF, tid - 256);
      }
      // qs (fq . z) over an eighth of the features (the last two quarters; at
      // FP = 32 waves 4 and 5 take a quarter each; none at FP = 256)
      constexpr int NE = FP >= 64 ? FP / 8 : 8;
      if constexpr (FP < 256) {
        if (const int f0 = FP / 2 + (wave - 4) * NE; f0 < FP)
          qz_part<NE>(fq_l, PF, zs, qs, qz + 64 * (wave - 2), lane, f0);
        else
          qz[64 * (wave - 2) + lane] = 0.f;
      }
    }
    // X = S dy^T for this wave's jobs, and qs fq . X per query
    f32x16 X[Cfg::XJ];
#pragma unroll
    for (int j = 0; j < Cfg::XJ; ++j) {
      int ft, hq;
      X[j] = zero16();
      if (x_job(j, ft, hq)) {
        const int q = hq * 32 + col;
        f32x16 x = zero16();
        if constexpr (SREG) {
          x = mfma_chain<DP / 16, PIPE>(
              x, [&](int kb) { return acc_operand(St[(j >> 1) * NDT + (kb >> 1)], kb & 1); },
              [&](int kb) { return row_operand_acc(dy_l, PD, q, 16 * kb, h); });
        } else {
          x = mfma_chain<DP / 16, PIPE>(
              x, [&](int kb) { return row_operand(s_l, PD, ft * 32 + col, 16 * kb, h); },
              [&](int kb) { return row_operand(dy_l, PD, q, 16 * kb, h); });
        }
        X[j] = x;
        float s = 0.f;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const bf16x4 f4 = *reinterpret_cast<const bf16x4*>(fq_l + q * PF + ft * 32 + 8 * g4 + 4 * h);
#pragma unroll
          for (int e = 0; e < 4; ++e) s += to_f32(f4[e]) * x[4 * g4 + e];
        }
        s += xhalf(s);
        if (h == 0) nx[ft * 64 + q] = s * qs[q];
      }
    }
    if (wave >= 4) issue(set, n + DEPTH);
    __syncthreads();
    // ---- phase 2: den, delta, dad fragments (waves 0-3) ------------------------
    if (live) {
      float den, delta;
      if constexpr (EXT) {
        const bool ok = t0 + qi < L;
        den = ok ? den_out[offL + t0 + qi] : 0.f;
        delta = ok ? delta_out[offL + t0 + qi] : 0.f;
      } else {
        den = ra[qi] + ra[64 + qi] + qz[qi] + qz[64 + qi] + qz[128 + qi] + qz[192 + qi];
        if constexpr (FP < 256) den += qz[256 + qi] + qz[320 + qi];
        float num = rav[qi] + rav[64 + qi];
#pragma unroll
        for (int ft = 0; ft < NFT; ++ft) num += nx[ft * 64 + qi];
        delta = num / fmaxf(den, TINY);
      }
      const float dcl = fmaxf(den, TINY);
      const float inv = 1.f / dcl;
      bf16x8 d8[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) d8[r >> 3][r & 7] = to_bf16((vdy[r] - delta) * inv * dec[r]);
      fr[(qt * 4 + kt * 2 + 0) * 64 + lane] = d8[0];
      fr[(qt * 4 + kt * 2 + 1) * 64 + lane] = d8[1];
      if (kt == 0 && h == 0) {
        dens[qi] = den;
        dels[qi] = delta;
        if (!EXT && t0 + qi < L) {
          den_out[offL + t0 + qi] = den;
          delta_out[offL + t0 + qi] = delta;
        }
      }
    }
    // z entering chunk n + 1, by waves 4-7, which have no phase-2 work
    const float r_n = rdec[0];
    if (tid >= 256) z_update<FP>(zb + FP * ((n + 1) & 1), zs, zp, r_n, tid - 256);
    __syncthreads();
    // ---- phase 3: dfq and fq . dfq for the X jobs; S^T update ------------------
#pragma unroll
    for (int j = 0; j < Cfg::XJ; ++j) {
      int ft, hq;
      if (x_job(j, ft, hq)) {
        const int q = hq * 32 + col;
        f32x16 g = zero16();
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)   // queries 0-31 have no keys in blocks 2, 3
          if (hq == 1 || kb < 2)
            g = mfma(tr_operand(fk_l, PF, 16 * kb, ft * 32, lane), fr[(hq * 4 + kb) * 64 + lane], g);
        const float dcl = fmaxf(dens[q], TINY);
        const float qsd = qs[q] / dcl;
        const float delta = dels[q];
        const int tok = t0 + q;
        float ps = 0.f;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int f0 = ft * 32 + 8 * g4 + 4 * h;
          const bf16x4 f4 = *reinterpret_cast<const bf16x4*>(fq_l + q * PF + f0);
          const f32x4 z4 = *reinterpret_cast<const f32x4*>(zs + f0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g4 + e;
            g[r] += qsd * (X[j][r] - z4[e] * delta);
            ps += to_f32(f4[e]) * g[r];
          }
        }
        ps += xhalf(ps);
        if (h == 0) pp[ft * 64 + q] = tok < L ? ps : 0.f;
        store_acc_row<OutT>(dfq + offF, tok, ft * 32, L, F, vecF, g, 1.f, h);
      }
    }
    // S^T <- r S^T + V^T K~ for the owned tiles
#pragma unroll
    for (int i = 0; i < Cfg::S_OWN; ++i) {
      int ft, dt;
      if (s_tile(i, ft, dt)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) St[i][r] *= r_n;
        St[i] = mfma_chain<4, PIPE>(
            St[i], [&](int kb) { return tr_operand(v_l, PD, 16 * kb, dt * 32, lane); },
            [&](int kb) { return tr_operand(kt_l, PF, 16 * kb, ft * 32, lane); });
      }
    }
    __syncthreads();
    // ---- next chunk into LDS; fq . dfq of this chunk; publish S --------------------
    if (wave == PW && t0 + lane < L) {
      float s = 0.f;
#pragma unroll
      for (int ft = 0; ft < NFT; ++ft) s += pp[ft * 64 + lane];
      p_out[offL + t0 + lane] = s;
    }
    if (n + 1 < n1) stage(std::integral_constant<int, (S + 1) % DEPTH>{});
    publish();
    __syncthreads();
  };
  for (int n = n0; n < n1; n += DEPTH) {
    step(SET0, n);
    if constexpr (DEPTH == 2)
      if (n + 1 < n1) step(SET1, n + 1);
  }
}

template <int FP, int DP, typename OutT, bool VEC, bool EXT, bool FOLD = false>
__global__ __launch_bounds__(B_THREADS, 1) void gla_bwd_dq_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, const bf16* __restrict__ dy, OutT* __restrict__ dfq,
    float* __restrict__ den_out, float* __restrict__ delta_out, float* __restrict__ p_out,
    const float* __restrict__ seg_state, int H, int L, int F, int D, int gate, int G,
    int cps, int M, int KG, int xper, int nxcd, int nblk, const float* __restrict__ seg_lam) {
  gla_bwd_dq_body<FP, DP, OutT, VEC, EXT, FOLD>(fq, fk, v, log_gamma, dy, dfq, den_out, delta_out,
                                                 p_out, seg_state, H, L, F, D, gate, G, cps, M,
                                                 KG, xper, nxcd, nblk, seg_lam);
}

// ============================================================================
// per-token scalars of the reverse walks: the gate scan of a chunk plus
// den (clamped), delta, p and Q^ scale qs/den, by one wave (lane = token)
// one token's gate value (raw, see gate_scan), den, delta and p, as the
// reverse walks load them; ok: the token is inside L
struct TokScalars {
  float g, den, delta, p;
  bool ok;
};

// ============================================================================
__device__ __forceinline__ void bwd_scalars(const TokScalars& sc, int gate, int lane,
                                            float* lgs, float* qs, float* ks, float* r,
                                            float* invd, float* dels, float* ps, float* qh,
                                            float* dw, float* gz = nullptr) {
  const float den = sc.den, delta = sc.delta, p = sc.p;
  gate_scan(sc.g, lane, lgs, qs, ks, r, gate, sc.ok);
  // d log_gamma -> the gate's own gradient (sigmoid(-z) for a logit, else 1)
  if (gz) gz[lane] = (gate & GATE_LOGIT) ? sigmoid_neg(sc.g) : 1.f;
  const float inv = 1.f / fmaxf(den, TINY);
  const float qhv = qs[lane] * inv;   // Q^_i = fq_i qs_i / den_i
  invd[lane] = inv;
  dels[lane] = delta;
  if (ps) ps[lane] = p;
  qh[lane] = qhv;
  dw[lane] = qhv * delta;             // dz = sum_i fq_i (qs_i delta_i / den_i)
}

// bf16(x[t][c] * scale[t]) for a [64 x KP] row-major tile, as 16-byte items
// (the item layout of scale_rows), without column sums
template <int KP>
__device__ __forceinline__ void scale_rows_only(const bf16* tile, int pitch, const float* scale,
                                                uint4 (&out)[RowItems<KP>::N]) {
  using R = RowItems<KP>;
  const int cg = threadIdx.x % R::K8, r0 = threadIdx.x / R::K8;
#pragma unroll
  for (int i = 0; i < R::N; ++i) {
    const int t = r0 + R::RSTRIDE * i;
    const bf16x8 x = *reinterpret_cast<const bf16x8*>(tile + t * pitch + 8 * cg);
    out[i] = __builtin_bit_cast(uint4, scale8(x, scale[t]));
  }
}

__device__ __forceinline__ TokScalars load_scalars(const float* __restrict__ lgb,
                                                   const float* __restrict__ den_in,
                                                   const float* __restrict__ delta_in,
                                                   const float* __restrict__ p_in, size_t offL,
                                                   int t, int L) {
  TokScalars s;
  const bool ok = t < L;
  s.ok = ok;
  s.g = ok ? lgb[t] : 0.f;
  s.den = ok ? den_in[offL + t] : 1.f;
  s.delta = ok ? delta_in[offL + t] : 0.f;
  s.p = (ok && p_in) ? p_in[offL + t] : 0.f;
  return s;
}

// ============================================================================
// reverse segment pass: gradient state left by segment g > 0 walking
// backwards from zero
// ============================================================================
template <int FP, int DP>
struct BwdS : BwdCommon<FP, DP> {
  using B_ = BwdCommon<FP, DP>;
  static constexpr int C = B_::C, PF = B_::PF, PD = B_::PD;
  static constexpr int OFF_FQ = 0;
  static constexpr int OFF_DY = OFF_FQ + C * PF * 2;
  static constexpr int OFF_LG = OFF_DY + C * PD * 2;
  static constexpr int OFF_QS = OFF_LG + 64 * 4;
  static constexpr int OFF_KS = OFF_QS + 64 * 4;
  static constexpr int OFF_INV = OFF_KS + 64 * 4;
  static constexpr int OFF_DEL = OFF_INV + 64 * 4;
  static constexpr int OFF_QH = OFF_DEL + 64 * 4;
  static constexpr int OFF_DW = OFF_QH + 64 * 4;
  static constexpr int OFF_DZ = OFF_DW + 64 * 4;
  static constexpr int OFF_DZP = OFF_DZ + FP * 4;
  static constexpr int OFF_R = OFF_DZP + 2048 * 4;        // 2048 partial sums (column_sums)
  static constexpr int BYTES = OFF_R + 16;
  static_assert(BYTES <= 80 * 1024, "LDS budget: two workgroups per CU");
};

template <int FP, int DP, bool VEC>
__global__ __launch_bounds__(256, 2) void gla_bwd_state_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ dy, const float* __restrict__ log_gamma,
    const float* __restrict__ den_in, const float* __restrict__ delta_in,
    float* __restrict__ seg_state, float* __restrict__ seg_logdecay, int H, int L, int F, int D,
    int gate, int G, int cps) {
  using Cfg = BwdS<FP, DP>;
  constexpr int C = Cfg::C, PF = Cfg::PF, PD = Cfg::PD;
  constexpr int NFT = Cfg::NFT, NDT = Cfg::NDT, NTILE = NFT * NDT, TPW = (NTILE + 3) / 4;
  extern __shared__ __align__(16) char smem[];
  bf16* fq_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQ);
  bf16* dy_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_DY);
  float* lgs = reinterpret_cast<float*>(smem + Cfg::OFF_LG);
  float* qs = reinterpret_cast<float*>(smem + Cfg::OFF_QS);
  float* ks = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  float* invd = reinterpret_cast<float*>(smem + Cfg::OFF_INV);
  float* dels = reinterpret_cast<float*>(smem + Cfg::OFF_DEL);
  float* qh = reinterpret_cast<float*>(smem + Cfg::OFF_QH);
  float* dw = reinterpret_cast<float*>(smem + Cfg::OFF_DW);
  float* dzs = reinterpret_cast<float*>(smem + Cfg::OFF_DZ);
  float* dzp = reinterpret_cast<float*>(smem + Cfg::OFF_DZP);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  const int bh = blockIdx.x / (G - 1), seg = 1 + blockIdx.x % (G - 1);
  const int NT = (L + C - 1) / C;
  const int n0 = seg * cps, n1 = min(NT, n0 + cps);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const bool vecF = VEC || (F & 7) == 0, vecD = VEC || (D & 7) == 0;
  const size_t offF = (size_t)bh * L * F, offD = (size_t)bh * L * D, offL = (size_t)bh * L;
  const float* lgb = log_gamma + (size_t)((gate & GATE_PER_HEAD) ? bh : bh / H) * L;

  f32x16 dS[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) dS[i] = zero16();
  for (int f = tid; f < FP; f += 256) dzs[f] = 0.f;
  float lam = 0.f;

  uint4 rq[Cfg::NLF], rd[Cfg::NLD];
  TokScalars sc;
  load_chunk<FP>(rq, fq + offF, (n1 - 1) * C, L, F, vecF);
  load_chunk<DP>(rd, dy + offD, (n1 - 1) * C, L, D, vecD);
  sc = load_scalars(lgb, den_in, delta_in, nullptr, offL, (n1 - 1) * C + lane, L);
  store_chunk<FP>(rq, fq_l, PF);
  store_chunk<DP>(rd, dy_l, PD);
  if (wave == 0)
    bwd_scalars(sc, gate, lane, lgs, qs, ks, rdec, invd, dels, nullptr, qh, dw);
  __syncthreads();

  for (int n = n1 - 1; n >= n0; --n) {
    const bool more = n - 1 >= n0;
    if (more) {
      load_chunk<FP>(rq, fq + offF, (n - 1) * C, L, F, vecF);
      load_chunk<DP>(rd, dy + offD, (n - 1) * C, L, D, vecD);
      sc = load_scalars(lgb, den_in, delta_in, nullptr, offL, (n - 1) * C + lane, L);
    }
    // dz partials sum_i fq_i (qh_i delta_i)
    column_sums<FP, false>(fq_l, PF, dw, dzp);
    __syncthreads();
    const float r_n = rdec[0];
    if (wave == 0) lam += rdec[1];
    // dS += Q^T dy, Q^ = bf16(qh fq) formed in registers.  Tile ti = wave + 4 i
    // has f-tile ti % NFT: one f-tile for all of a wave's tiles when NFT
    // divides 4, two (i even, i odd) when NFT = 8, so the scaled operands are
    // formed once per f-tile
    constexpr int NQF = NFT <= 4 ? 1 : 2;
    static_assert(NFT <= 8 && (NFT <= 4 || NFT % 4 == 0), "state pass f-tiles");
    bf16x8 qf[NQF][4];
#pragma unroll
    for (int j = 0; j < NQF; ++j)
      if (wave + 4 * j < NTILE)
#pragma unroll
        for (int qb = 0; qb < 4; ++qb)
          qf[j][qb] = tr_operand_scaled(fq_l, PF, 16 * qb, ((wave + 4 * j) % NFT) * 32, lane, qh);
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int ti = wave + 4 * i;
      if (ti < NTILE) {
        const int dt = ti / NFT;
#pragma unroll
        for (int r = 0; r < 16; ++r) dS[i][r] *= r_n;
#pragma unroll
        for (int qb = 0; qb < 4; ++qb)
          dS[i] = mfma(qf[i % NQF][qb], tr_operand(dy_l, PD, 16 * qb, dt * 32, lane), dS[i]);
      }
    }
    __syncthreads();
    if (more) {
      store_chunk<FP>(rq, fq_l, PF);
      store_chunk<DP>(rd, dy_l, PD);
      if (wave == 0)
        bwd_scalars(sc, gate, lane, lgs, qs, ks, rdec, invd, dels, nullptr, qh,
                    dw);
    }
    if (tid < FP) dzs[tid] = dzs[tid] * r_n + sum_parts<FP>(dzp, tid);
    __syncthreads();
  }
  float* out = seg_state + ((size_t)bh * G + seg) * Cfg::SEG;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int ti = wave + 4 * i;
    if (ti < NTILE) {
      const int ft = ti % NFT, dt = ti / NFT;
#pragma unroll
      for (int r = 0; r < 16; ++r) out[(ft * 32 + acc_row(r, h)) * DP + dt * 32 + col] = dS[i][r];
    }
  }
  for (int f = tid; f < FP; f += 256) out[FP * DP + f] = dzs[f];
  if (tid == 0) seg_logdecay[(size_t)bh * G + seg] = lam;
}

// ============================================================================
// kernel B: reverse walk -> dv, dfk, dG = p - fk . dfk
//
// Eight waves share one chunk (the LDS of a chunk leaves room for one
// workgroup per CU, so the second wave per SIMD comes from inside it):
//   phase 1  wave (kind, qt, kt): kind 0 the score tile s -> a/den, kind 1 the
//            dy.v^T tile -> dad (both need only their own tile).  The tiles of
//            keys 32-63 x queries 0-31 are causally zero: their two waves
//            form the dz partials instead, and the phase-2 products skip
//            those zero fragments;
//   phase 2  dv jobs (d-tile, key half) contract dS over f from the published
//            bf16 dS^T tile; dS tiles (f-tile, d-tile) are spread over the
//            waves' accumulators and updated with Q^T dy, Q^ = bf16(qh fq)
//            formed in registers from fq's transpose reads (the reference
//            rounds the same operand, src/kernels/gla.py:104-132); dfk jobs
//            (f-tile, key half) contract dS^T over d;
//   tail     dG, publish dS^T, stage the prefetched chunk, dz update.
// ============================================================================
template <int FP, int DP>
struct BwdB : BwdCommon<FP, DP> {
  using B_ = BwdCommon<FP, DP>;
  static constexpr int C = B_::C, PF = B_::PF, PD = B_::PD, NFT = B_::NFT, NDT = B_::NDT;
  // dz partial sums per feature (4 at FP = 256, where the chunk's LDS is tightest)
  static constexpr int ZP = FP >= 256 ? 4 : 8;
  static constexpr int S_OWN = (NFT * NDT + B_WAVES - 1) / B_WAVES;   // dS tiles per wave
  static constexpr int DV_JOBS = 2 * NDT, DFK_JOBS = 2 * NFT;
  static constexpr int DV_OWN = (DV_JOBS + B_WAVES - 1) / B_WAVES;
  static constexpr int DFK_OWN = (DFK_JOBS + B_WAVES - 1) / B_WAVES;
  static constexpr int DEPTH = 1;   // as in BwdA
  // chunk tiles per thread (16-byte items), rounded up; the last may be partial
  static constexpr int NLF = (C * FP / 8 + B_THREADS - 1) / B_THREADS;
  static constexpr int NLD = (C * DP / 8 + B_THREADS - 1) / B_THREADS;
  static constexpr int OFF_FQ = 0;
  static constexpr int OFF_FK = OFF_FQ + C * PF * 2;
  static constexpr int OFF_V = OFF_FK + C * PF * 2;
  static constexpr int OFF_DY = OFF_V + C * PD * 2;
  static constexpr int OFF_DST = OFF_DY + C * PD * 2;     // dS^T [DP][PF] bf16
  static constexpr int OFF_FA = OFF_DST + DP * PF * 2;    // a/den fragments [2 kt][4 qb][64]
  static constexpr int OFF_FD = OFF_FA + 2 * 4 * 64 * 16; // dad fragments
  static constexpr int OFF_PK = OFF_FD + 2 * 4 * 64 * 16; // [NFT][64] fk . dfk partials
  static constexpr int OFF_INV = OFF_PK + NFT * 64 * 4;   // per-token scalars, [2][64] by parity
  static constexpr int OFF_DEL = OFF_INV + 2 * 64 * 4;
  static constexpr int OFF_P = OFF_DEL + 2 * 64 * 4;
  static constexpr int OFF_QH = OFF_P + 2 * 64 * 4;
  static constexpr int OFF_DW = OFF_QH + 2 * 64 * 4;
  static constexpr int OFF_LG = OFF_DW + 2 * 64 * 4;
  static constexpr int OFF_QS = OFF_LG + 64 * 4;
  static constexpr int OFF_KS = OFF_QS + 64 * 4;
  static constexpr int OFF_DZ = OFF_KS + 64 * 4;
  static constexpr int OFF_DZP = OFF_DZ + FP * 4;
  static constexpr int OFF_GZ = OFF_DZP + ZP * FP * 4;   // [2][64] d log_gamma scales
  static constexpr int OFF_R = OFF_GZ + 2 * 64 * 4;
  static constexpr int BYTES = OFF_R + 16;
  static constexpr int LB = BYTES <= 80 * 1024 ? 2 : 1;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
};

template <int FP, int DP, typename OutT, bool VEC, bool FOLD = false>
__device__ __forceinline__ void gla_bwd_dkv_body(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, const bf16* __restrict__ dy,
    const float* __restrict__ den_in, const float* __restrict__ delta_in,
    const float* __restrict__ p_in, OutT* __restrict__ dfk, OutT* __restrict__ dv,
    float* __restrict__ dG, float* __restrict__ csum, float* __restrict__ dlg_direct,
    const float* __restrict__ seg_state, int H,
    int L, int F, int D, int gate, int G, int cps, int M, int KG, int xper, int nxcd,
    int nblk, const float* __restrict__ seg_lam, int rev) {
  using Cfg = BwdB<FP, DP>;
  constexpr int C = Cfg::C, PF = Cfg::PF, PD = Cfg::PD;
  constexpr int NFT = Cfg::NFT, NDT = Cfg::NDT, ZP = Cfg::ZP;
  extern __shared__ __align__(16) char smem[];
  bf16* fq_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQ);
  bf16* fk_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FK);
  bf16* v_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_V);
  bf16* dy_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_DY);
  bf16* dst_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_DST);
  bf16x8* fa = reinterpret_cast<bf16x8*>(smem + Cfg::OFF_FA);
  bf16x8* fd = reinterpret_cast<bf16x8*>(smem + Cfg::OFF_FD);
  float* pk = reinterpret_cast<float*>(smem + Cfg::OFF_PK);
  float* invd = reinterpret_cast<float*>(smem + Cfg::OFF_INV);
  float* dels = reinterpret_cast<float*>(smem + Cfg::OFF_DEL);
  float* ps = reinterpret_cast<float*>(smem + Cfg::OFF_P);
  float* qh = reinterpret_cast<float*>(smem + Cfg::OFF_QH);
  float* dw = reinterpret_cast<float*>(smem + Cfg::OFF_DW);
  float* lgs = reinterpret_cast<float*>(smem + Cfg::OFF_LG);
  float* qs = reinterpret_cast<float*>(smem + Cfg::OFF_QS);
  float* ks = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  float* dzs = reinterpret_cast<float*>(smem + Cfg::OFF_DZ);
  float* dzp = reinterpret_cast<float*>(smem + Cfg::OFF_DZP);
  float* gz = reinterpret_cast<float*>(smem + Cfg::OFF_GZ);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  // a workgroup walks M consecutive segments (seg0 .. seg0 + M - 1) in reverse,
  // entering with the state that flows into the last of them
  const int nwg = G / M;
  int blk;
  if (!walk_block(xper, nxcd, nblk, blk, rev != 0)) return;
  const int bh = blk / nwg, seg0 = (blk % nwg) * M, seg = seg0 + M - 1;
  const int NT = (L + C - 1) / C;
  const int n0 = seg0 * cps, n1 = min(NT, n0 + M * cps);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const bool vecF = VEC || (F & 7) == 0, vecD = VEC || (D & 7) == 0;
  const size_t offF = (size_t)bh * L * F, offD = (size_t)bh * L * D, offL = (size_t)bh * L;
  // fk and v of the kv head of this query head (KG query heads share one)
  const size_t offFk = (size_t)(bh / KG) * L * F, offDv = (size_t)(bh / KG) * L * D;
  const float* lgb = log_gamma + (size_t)((gate & GATE_PER_HEAD) ? bh : bh / H) * L;
  // the gradient state entering segment seg from the right: its scanned
  // record, or (FOLD) the local records of segments G - 1 .. seg + 1 folded
  // here (their total log decays at seg_lam)
  const float* st =
      G > 1 ? seg_state + ((size_t)bh * G + (FOLD ? 0 : seg)) * Cfg::SEG : nullptr;

  // this wave's dS tiles t = wave + 8 i: f-tile t % NFT, d-tile t / NFT
  // (lane = d column, registers = f rows)
  f32x16 dS[Cfg::S_OWN];
  if constexpr (FOLD) {   // folded in LDS, before the first chunk is staged there
    static_assert(Cfg::SEG * 4 <= Cfg::BYTES, "a folded record fits the chunk's LDS");
    float* fold_l = reinterpret_cast<float*>(smem);
    const bool any = seg < G - 1;
    if (any)
      fold_records<B_THREADS, Cfg::SEG, 160>(fold_l, st, seg_lam + (size_t)bh * G, G - 1, -1,
                                             G - 1 - seg);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < Cfg::S_OWN; ++i) {
      dS[i] = zero16();
      const int t = wave + B_WAVES * i;
      if (any && t < NFT * NDT) {
        const int ft = t % NFT, dt = t / NFT;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          dS[i][r] = fold_l[(ft * 32 + acc_row(r, h)) * DP + dt * 32 + col];
      }
    }
    static_assert(FP <= B_THREADS, "one dz element per thread");
    const float zv = any && tid < FP ? fold_l[FP * DP + tid] : 0.f;
    __syncthreads();   // read before the LDS is reused
    if (tid < FP) dzs[tid] = zv;
  } else {
#pragma unroll
    for (int i = 0; i < Cfg::S_OWN; ++i) {
      dS[i] = zero16();
      const int t = wave + B_WAVES * i;
      if (st && t < NFT * NDT) {
        const int ft = t % NFT, dt = t / NFT;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          dS[i][r] = st[(ft * 32 + acc_row(r, h)) * DP + dt * 32 + col];
      }
    }
    for (int f = tid; f < FP; f += B_THREADS) dzs[f] = st ? st[FP * DP + f] : 0.f;
  }

  // publish the owned dS tiles as bf16 dS^T [d][f] (4 consecutive f per store)
  auto publish = [&]() {
#pragma unroll
    for (int i = 0; i < Cfg::S_OWN; ++i) {
      const int t = wave + B_WAVES * i;
      if (t < NFT * NDT) {
        const int ft = t % NFT, d = (t / NFT) * 32 + col;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          bf16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = to_bf16(dS[i][4 * g4 + e]);
          *reinterpret_cast<bf16x4*>(dst_l + d * PF + ft * 32 + 8 * g4 + 4 * h) = o;
        }
      }
    }
  };

  // per-chunk single-wave work goes to waves whose tail is otherwise light:
  // the token scalars to wave 3, dG to wave 2, the dz update to waves 4 and up
  constexpr int SCW = 3, DGW = 2;
  // DEPTH register sets: while chunk n computes, chunks n-1 .. n-DEPTH are in flight
  constexpr int DEPTH = Cfg::DEPTH;
  uint4 rq[DEPTH][Cfg::NLF], rk[DEPTH][Cfg::NLF], rv[DEPTH][Cfg::NLD], rd[DEPTH][Cfg::NLD];
  TokScalars sc[DEPTH];
  auto issue = [&](auto set, int n) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    if (n >= n0) {
      load_tile8<FP>(rq[S], fq + offF, n * C, L, F, vecF);
      load_tile8<FP>(rk[S], fk + offFk, n * C, L, F, vecF);
      load_tile8<DP>(rv[S], v + offDv, n * C, L, D, vecD);
      load_tile8<DP>(rd[S], dy + offD, n * C, L, D, vecD);
      if (wave == SCW) sc[S] = load_scalars(lgb, den_in, delta_in, p_in, offL, n * C + lane, L);
    }
  };
  // chunk n's tiles and per-token scalars (scalars into the buffers of parity n & 1)
  auto stage = [&](auto set, int n) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    store_tile8<FP>(rq[S], fq_l, PF);
    store_tile8<FP>(rk[S], fk_l, PF);
    store_tile8<DP>(rv[S], v_l, PD);
    store_tile8<DP>(rd[S], dy_l, PD);
    const int b = n & 1;
    if (wave == SCW)
      bwd_scalars(sc[S], gate, lane, lgs, qs, ks, rdec, invd + 64 * b, dels + 64 * b,
                  ps + 64 * b, qh + 64 * b, dw + 64 * b, dlg_direct ? gz + 64 * b : nullptr);
  };
  issue(SET0, n1 - 1);
  if constexpr (DEPTH == 2) issue(SET1, n1 - 2);
  stage(SET0, n1 - 1);
  publish();
  __syncthreads();

  const int kind = wave >> 2, qt = (wave >> 1) & 1, kt = wave & 1;   // phase-1 tile
  const int ki = kt * 32 + col;                                       // its key (lane)
  // waves 1 and 5 hold the causally zero tiles (kt = 1, qt = 0): they form the
  // dz partial sums instead, as threads a = 0 .. 127
  const bool stager = kt == 1 && qt == 0;
  const int a = (kind << 6) + lane;
  // with dlg_direct (a per-head gate, one segment: this walk sees all of its
  // row), d log_gamma is written here; dlg_after sums dG of the chunks walked
  float dlg_after = 0.f;
  // chunk n is in LDS and register set `set` is free; the next set holds chunk n-1
  auto step = [&](auto set, int n) __attribute__((always_inline)) {
    constexpr int S = decltype(set)::value;
    const int t0 = n * C;
    const int cur = n & 1;
    const float* invc = invd + 64 * cur;
    const float* delsc = dels + 64 * cur;
    const float* qhc = qh + 64 * cur;
    const float* dwc = dw + 64 * cur;
    // waves 0-3 load the next chunk of the walk now, waves 4-7 once their
    // phase-1 work is done: issued together, the later waves' loads waited for
    // free slots in the CU's memory queue and held back their phase-1 products
    if (wave < 4) issue(set, n - DEPTH);
    // ---- phase 1: one 32x32 tile (queries x keys) of s or dy v^T per wave ----
    if (!stager) {
      f32x16 acc = zero16();
      if (kind == 0) {
        acc = mfma_chain<FP / 16, 2>(
            acc, [&](int kb) { return row_operand(fq_l, PF, qt * 32 + col, 16 * kb, h); },
            [&](int kb) { return row_operand(fk_l, PF, ki, 16 * kb, h); });
      } else {
        acc = mfma_chain<DP / 16, 2>(
            acc, [&](int kb) { return row_operand(dy_l, PD, qt * 32 + col, 16 * kb, h); },
            [&](int kb) { return row_operand(v_l, PD, ki, 16 * kb, h); });
      }
      const float lgk = lgs[ki];
      bf16x8 o8[2];
      // kind is uniform per wave: the test sits outside the element loops, so
      // each wave runs one straight-line loop instead of a branch per element
      if (kind == 0) {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int q0 = qt * 32 + 8 * g4 + 4 * h;   // queries of registers 4 g4 .. +4
          const f32x4 lq = *reinterpret_cast<const f32x4*>(lgs + q0);
          const f32x4 iv = *reinterpret_cast<const f32x4*>(invc + q0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g4 + e;
            const float dec = ki <= q0 + e ? fexp(lq[e] - lgk) : 0.f;
            o8[r >> 3][r & 7] = to_bf16(to_f32(to_bf16(acc[r] * dec)) * iv[e]);   // a / den
          }
        }
      } else {
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int q0 = qt * 32 + 8 * g4 + 4 * h;
          const f32x4 lq = *reinterpret_cast<const f32x4*>(lgs + q0);
          const f32x4 iv = *reinterpret_cast<const f32x4*>(invc + q0);
          const f32x4 dl = *reinterpret_cast<const f32x4*>(delsc + q0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g4 + e;
            const bool c = ki <= q0 + e;
            const float dec = c ? fexp(lq[e] - lgk) : 0.f;
            o8[r >> 3][r & 7] = to_bf16(c ? (acc[r] - dl[e]) * iv[e] * dec : 0.f);   // dad
          }
        }
      }
      bf16x8* frag = kind == 0 ? fa : fd;
      frag[(kt * 4 + qt * 2 + 0) * 64 + lane] = o8[0];
      frag[(kt * 4 + qt * 2 + 1) * 64 + lane] = o8[1];
    }
    // dz partials: part p sums fq_t (qh_t delta_t) over tokens [8 p, 8 p + 8)
    {
      constexpr int K8 = FP / 8;
      static_assert(ZP * K8 <= 128, "dz partials: one per staging thread");
      if (stager && a < ZP * K8) {
        const int c8 = 8 * (a % K8), part = a / K8;
        float za[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < C / ZP; ++j) {
          const int t = part * (C / ZP) + j;
          const bf16x8 x = *reinterpret_cast<const bf16x8*>(fq_l + t * PF + c8);
          const float w = dwc[t];
#pragma unroll
          for (int e = 0; e < 8; ++e) za[e] += to_f32(x[e]) * w;
        }
        float* dst = dzp + part * FP + c8;
        *reinterpret_cast<f32x4*>(dst) = f32x4{za[0], za[1], za[2], za[3]};
        *reinterpret_cast<f32x4*>(dst + 4) = f32x4{za[4], za[5], za[6], za[7]};
      }
    }
    if (wave >= 4) issue(set, n - DEPTH);
    __syncthreads();
    const float r_n = rdec[0];
    // ---- phase 2: dv jobs from the published dS^T -----------------------------
#pragma unroll
    for (int i = 0; i < Cfg::DV_OWN; ++i) {
      const int job = wave + B_WAVES * i;
      if (job < Cfg::DV_JOBS) {
        const int dt = job >> 1, hk = job & 1;
        const int key = hk * 32 + col;
        // dv_t = ks_t (fk_t dS) + sum_i (a_it / den_i) dy_i: the row scale of
        // K~ = fk ks multiplies the fp32 product
        f32x16 g = zero16();
        g = mfma_chain<FP / 16, 2>(
            g, [&](int kb) { return row_operand(dst_l, PF, dt * 32 + col, 16 * kb, h); },
            [&](int kb) { return row_operand(fk_l, PF, key, 16 * kb, h); });
        const float ksv = ks[key];
#pragma unroll
        for (int r = 0; r < 16; ++r) g[r] *= ksv;
#pragma unroll
        for (int qb = 0; qb < 4; ++qb)   // keys 32-63 have no queries in blocks 0, 1
          if (hk == 0 || qb >= 2)
            g = mfma(tr_operand(dy_l, PD, 16 * qb, dt * 32, lane), fa[(hk * 4 + qb) * 64 + lane], g);
        store_acc_row<OutT>(dv + offD, t0 + key, dt * 32, L, D, vecD, g, 1.f, h);
      }
    }
    // dS <- r_n dS + Q^T dy for the owned tiles, Q^ = bf16(qh fq): the owned
    // tiles t = wave + 8 i share the f-tile wave % NFT (8 is a multiple of
    // NFT), so its four scaled operands are formed once per chunk
    static_assert(B_WAVES % NFT == 0, "owned dS tiles share one f-tile");
    if (wave < NFT * NDT) {
      const int ft = wave % NFT;
      bf16x8 qf[4];
#pragma unroll
      for (int qb = 0; qb < 4; ++qb)
        qf[qb] = tr_operand_scaled(fq_l, PF, 16 * qb, ft * 32, lane, qhc);
#pragma unroll
      for (int i = 0; i < Cfg::S_OWN; ++i) {
        const int t = wave + B_WAVES * i;
        if (t < NFT * NDT) {
          const int dt = t / NFT;
#pragma unroll
          for (int r = 0; r < 16; ++r) dS[i][r] *= r_n;
          dS[i] = mfma_chain<4, 2>(
              dS[i], [&](int qb) { return qf[qb]; },
              [&](int qb) { return tr_operand(dy_l, PD, 16 * qb, dt * 32, lane); });
        }
      }
    }
    // ---- dfk jobs (f-tile, key half), from the published dS^T -----------------
#pragma unroll
    for (int i = 0; i < Cfg::DFK_OWN; ++i) {
      // the other key half than this wave's dv job: a SIMD's two waves then
      // carry one short (keys 32-63) and one long job of each kind
      const int job = (wave ^ 1) + B_WAVES * i;
      if (job < Cfg::DFK_JOBS) {
        const int ft = job >> 1, hk = job & 1;
        const int key = hk * 32 + col;
        f32x16 x = zero16(), g = zero16();
        x = mfma_chain<DP / 16, 2>(
            x, [&](int kb) { return tr_operand_c(dst_l, PF, 16 * kb, ft * 32, lane); },
            [&](int kb) { return row_operand(v_l, PD, key, 16 * kb, h); });
#pragma unroll
        for (int qb = 0; qb < 4; ++qb)   // keys 32-63 have no queries in blocks 0, 1
          if (hk == 0 || qb >= 2)
            g = mfma(tr_operand(fq_l, PF, 16 * qb, ft * 32, lane), fd[(hk * 4 + qb) * 64 + lane], g);
        const float ksv = ks[key];
        const int tok = t0 + key;
        float pks = 0.f;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          const int f0 = ft * 32 + 8 * g4 + 4 * h;
          const bf16x4 k4 = *reinterpret_cast<const bf16x4*>(fk_l + key * PF + f0);
          const f32x4 z4 = *reinterpret_cast<const f32x4*>(dzs + f0);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * g4 + e;
            g[r] += ksv * (x[r] - z4[e]);
            pks += to_f32(k4[e]) * g[r];
          }
        }
        pks += xhalf(pks);
        if (h == 0) pk[ft * 64 + key] = pks;
        store_acc_row<OutT>(dfk + offF, tok, ft * 32, L, F, vecF, g, 1.f, h);
      }
    }
    __syncthreads();
    // ---- dG of this chunk and its sum; publish dS; previous chunk; dz update ---
    if (wave == DGW) {
      float g = 0.f;
      if (t0 + lane < L) {
        float s = 0.f;
#pragma unroll
        for (int ft = 0; ft < NFT; ++ft) s += pk[ft * 64 + lane];
        g = ps[64 * cur + lane] - s;
        if (!dlg_direct) dG[offL + t0 + lane] = g;
      }
      if (dlg_direct) {
        // d log_gamma of this chunk: the chunks after it are already summed
        const float suf = wave_suffix_sum(g, lane);
        if (t0 + lane < L) dlg_direct[offL + t0 + lane] = (dlg_after + suf) * gz[64 * cur + lane];
        dlg_after += __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(suf)));
      } else {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) g += __shfl_xor(g, off);
        if (lane == 0) csum[(size_t)bh * NT + n] = g;
      }
    }
    publish();
    if (n - 1 >= n0) stage(std::integral_constant<int, (S + 1) % DEPTH>{}, n - 1);
    for (int f = tid - 256; f >= 0 && f < FP; f += 256) {
      float za = dzs[f] * r_n;
#pragma unroll
      for (int p = 0; p < ZP; ++p) za += dzp[p * FP + f];
      dzs[f] = za;
    }
    __syncthreads();
  };
  for (int n = n1 - 1; n >= n0; n -= DEPTH) {
    step(SET0, n);
    if constexpr (DEPTH == 2)
      if (n - 1 >= n0) step(SET1, n - 1);
  }
}

template <int FP, int DP, typename OutT, bool VEC, bool FOLD = false>
__global__ __launch_bounds__(B_THREADS, (BwdB<FP, DP>::LB)) void gla_bwd_dkv_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, const bf16* __restrict__ dy,
    const float* __restrict__ den_in, const float* __restrict__ delta_in,
    const float* __restrict__ p_in, OutT* __restrict__ dfk, OutT* __restrict__ dv,
    float* __restrict__ dG, float* __restrict__ csum, float* __restrict__ dlg_direct,
    const float* __restrict__ seg_state, int H,
    int L, int F, int D, int gate, int G, int cps, int M, int KG, int xper, int nxcd,
    int nblk, const float* __restrict__ seg_lam, int rev) {
  gla_bwd_dkv_body<FP, DP, OutT, VEC, FOLD>(fq, fk, v, log_gamma, dy, den_in, delta_in, p_in, dfk,
                                            dv, dG, csum, dlg_direct, seg_state, H, L, F, D, gate,
                                            G, cps, M, KG, xper, nxcd, nblk, seg_lam, rev);
}

// One segment per (b, h): the dq walk and then the dkv walk of the same
// (b, h) in one workgroup.  The dkv walk starts on the chunks the dq walk
// read last, still in the caches, and needs only this workgroup's own den,
// delta and p rows (a workgroup-scope fence and barrier order them).
template <int FP, int DP, typename OutT, bool VEC>
__global__ __launch_bounds__(B_THREADS, 1) void gla_bwd_fused_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, const bf16* __restrict__ dy, OutT* __restrict__ dfq,
    OutT* __restrict__ dfk, OutT* __restrict__ dv, float* __restrict__ den,
    float* __restrict__ delta, float* __restrict__ p, float* __restrict__ dG,
    float* __restrict__ csum, float* __restrict__ dlg_direct, int H, int L, int F, int D,
    int gate, int cps, int KG, int xper, int nxcd, int nblk) {
  gla_bwd_dq_body<FP, DP, OutT, VEC, false>(fq, fk, v, log_gamma, dy, dfq, den, delta, p, nullptr,
                                            H, L, F, D, gate, 1, cps, 1, KG, xper, nxcd, nblk,
                                            nullptr);
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");
  __syncthreads();
  gla_bwd_dkv_body<FP, DP, OutT, VEC>(fq, fk, v, log_gamma, dy, den, delta, p, dfk, dv, dG, csum,
                                      dlg_direct, nullptr, H, L, F, D, gate, 1, cps, 1, KG, xper,
                                      nxcd, nblk, nullptr, 0);
}

// ============================================================================
// d log_gamma[row, j] = sum_{j' >= j} value[row, j'], value = dG of that (b, h)
// row (per-head gate) or its sum over the heads (per-token gate).  One wave
// per (row, 64-token chunk) and per workgroup, so the loads of a small grid
// spread over as many CUs as there are chunks; no barriers.  Lane t
// holds token t of the chunk summed over the heads; the chunk totals of the
// later chunks (lanes over chunks, summed over the heads) come in alongside.
// Loads go out in batches of BATCH buffer loads (zero past the end; BATCH
// is the number of heads summed, rounded up to 8, at most 16), the gate
// logit with the first batch; the sums over lanes are DPP scans.  Fixed
// order throughout.
// ============================================================================
constexpr int GATE_CHUNKS_PER_WG = 1;

template <int BATCH>
__global__ __launch_bounds__(64 * GATE_CHUNKS_PER_WG) void gla_gate_grad_kernel(
    const float* __restrict__ dG, const float* __restrict__ csum,
    const float* __restrict__ gate_in, float* __restrict__ dlg, int H, int L, int gate) {
  const int row = blockIdx.y, lane = threadIdx.x & 63;
  const int NT = (L + GLA_C - 1) / GLA_C;
  const int c = blockIdx.x * GATE_CHUNKS_PER_WG + (threadIdx.x >> 6);
  if (c >= NT) return;   // whole waves; nothing below synchronises across waves
  const int nsum = (gate & GATE_PER_HEAD) ? 1 : H;
  const rsrc_t src = make_rsrc(dG + (size_t)row * nsum * L, (size_t)nsum * L * 4);
  const rsrc_t cs = make_rsrc(csum + (size_t)row * nsum * NT, (size_t)nsum * NT * 4);
  const int j = c * GLA_C + lane;
  const size_t at = (size_t)row * L + j;
  // a buffer load (zero past the end, none without GATE_LOGIT): no branch
  // around it, so nothing waits for it before the batches go out
  const bool logit = (gate & GATE_LOGIT) != 0;
  const rsrc_t gz = make_rsrc(logit ? gate_in + (size_t)row * L : nullptr, logit ? (size_t)L * 4 : 0);
  const float z = bload_f32(gz, j < L ? (uint32_t)j * 4u : OOB);
  float val = 0.f, after = 0.f;
  for (int h0 = 0; h0 < nsum; h0 += BATCH) {
    float x[BATCH];
#pragma unroll
    for (int k = 0; k < BATCH; ++k)
      x[k] = bload_f32(src, (h0 + k < nsum && j < L) ? (uint32_t)((h0 + k) * L + j) * 4u : OOB);
    for (int c2 = c + 1 + lane; c2 - lane < NT; c2 += 64) {
      float y[BATCH];
#pragma unroll
      for (int k = 0; k < BATCH; ++k)
        y[k] = bload_f32(cs, (h0 + k < nsum && c2 < NT) ? (uint32_t)((h0 + k) * NT + c2) * 4u : OOB);
#pragma unroll
      for (int k = 0; k < BATCH; ++k) after += y[k];
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) val += x[k];
  }
  after = wave_prefix_sum(after);
  after = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(after), 63));
  val = wave_suffix_sum(val, lane);   // inclusive suffix sum over the chunk
  // GATE_LOGIT: the gradient of the logit z, d log_gamma * sigmoid(-z)
  if (j < L) dlg[at] = (gate & GATE_LOGIT) ? (after + val) * sigmoid_neg(z) : after + val;
}

// ============================================================================
// host launchers
// ============================================================================
static int gate_rows(int B, int H, int gate) { return (gate & GATE_PER_HEAD) ? B * H : B; }

// den, delta, p, dG [BH][L]; forward and reverse segment records; chunk sums
// of dG [BH][NT]
size_t gla_bwd_workspace(int B, int H, int L, int F, int D, int gate) {
  (void)gate;
  const int BH = B * H;
  int G, cps;
  gla_segments(BH, L, F, &G, &cps);
  const size_t NT = (L + GLA_C - 1) / GLA_C;
  return (4 * (size_t)BH * L + 2 * gla_segment_floats(BH, G, F, D) + (size_t)BH * NT) *
         sizeof(float);
}

// d log_gamma from dG and the per-chunk dG totals: one wave per (row,
// chunk), BATCH loads per batch (the heads summed, rounded up to 8, at most 16)
static hipError_t launch_gate_grad(const float* dG, const float* csum, const float* lg,
                                   float* dlg, int B, int H, int L, int gate, hipStream_t st) {
  const int nt = (L + GLA_C - 1) / GLA_C;
  const dim3 ggrid((nt + GATE_CHUNKS_PER_WG - 1) / GATE_CHUNKS_PER_WG, gate_rows(B, H, gate));
  const int nsum = (gate & GATE_PER_HEAD) ? 1 : H;
  auto kg = nsum == 1 ? gla_gate_grad_kernel<1>
          : nsum <= 8 ? gla_gate_grad_kernel<8>
          : gla_gate_grad_kernel<16>;
  hipLaunchKernelGGL(kg, ggrid, dim3(64 * GATE_CHUNKS_PER_WG), 0, st, dG, csum, lg, dlg, H, L,
                     gate);
  return hipGetLastError();
}

template <int FP, int DP, typename OutT, bool VEC>
static hipError_t launch_gla_bwd_t(const void* fq, const void* fk, const void* v, const float* lg,
                                   const void* dy, void* dfq, void* dfk, void* dv, float* dlg,
                                   int B, int H, int L, int F, int D, int gate, int KG,
                                   const float* fwd_ws, float* ws, const float* ext_den,
                                   const float* ext_delta, hipStream_t st) {
  const int BH = B * H;
  const size_t BHL = (size_t)BH * L;
  int G, cps;
  gla_segments(BH, L, F, &G, &cps);
  constexpr int SEG = SegRec<FP, DP>::SIZE;
  constexpr int LDS_A = BwdA<FP, DP>::BYTES, LDS_S = BwdS<FP, DP>::BYTES;
  constexpr int LDS_B = BwdB<FP, DP>::BYTES;
  // den and delta of the whole feature dimension, when given (ext_den), else
  // kernel A forms them into the workspace
  const bool ext = ext_den != nullptr;
  float* den = ext ? const_cast<float*>(ext_den) : ws;
  float* delta = ext ? const_cast<float*>(ext_delta) : ws + BHL;
  float* p = ws + 2 * BHL;
  float* dG = p + BHL;
  const size_t segf = gla_segment_floats(BH, G, F, D);
  float* own_fseg = dG + BHL;
  float* rseg = own_fseg + segf;
  float* csum = rseg + segf;
  const float* fseg = fwd_ws ? fwd_ws : own_fseg;   // the forward's records, when kept
  // the walks fold the segment records themselves (the state passes, here
  // and in the forward that kept them, leave them unscanned), or read the
  // scanned ones
  constexpr bool CAN_FOLD = gla_can_fold<FP, DP, VEC>();
  const bool fold = CAN_FOLD && !ext && gla_fold_segments(G);
  hipError_t e;
  if (G > 1 && !fwd_ws) {
    e = launch_gla_fwd_states(fk, v, lg, own_fseg, own_fseg + (size_t)BH * G * SEG, BH, H, L, F,
                              D, gate, G, cps, KG, fold, st);
    if (e != hipSuccess) return e;
  }
  // the walks take two segments per workgroup while that still gives one
  // workgroup per CU: fewer, longer walks
  const int M = (G % 2 == 0 && BH * G / 2 >= device_geom().cus) ? 2 : 1;
  const WalkGrid wg = walk_grid(BH * G / M, KG);
  const float* flam = fseg + (size_t)BH * G * SEG;
  // One segment per (b, h): the dq and dkv walks of a (b, h) run in one
  // workgroup, one after the other (gla_bwd_fused_kernel): one launch, and
  // the dkv walk starts on the chunks the dq walk read last, in every round
  // of workgroups (headline fwd+bwd 0.8808 -> 0.8628 ms, same bits).
  // a per-head gate in one segment: the reverse walk of (b, h) sees its whole
  // gate row and writes d log_gamma itself (no gate launch, no dG)
  const bool direct_dlg = (gate & GATE_PER_HEAD) && G == 1;
  if (G == 1 && !ext) {
    auto kf = gla_bwd_fused_kernel<FP, DP, OutT, VEC>;
    constexpr int LDS_F = LDS_A > LDS_B ? LDS_A : LDS_B;
    if ((e = ensure_lds<gla_bwd_fused_kernel<FP, DP, OutT, VEC>>(LDS_F)) != hipSuccess) return e;
    hipLaunchKernelGGL(kf, dim3(wg.grid), dim3(B_THREADS), LDS_F, st, (const bf16*)fq,
                       (const bf16*)fk, (const bf16*)v, lg, (const bf16*)dy, (OutT*)dfq,
                       (OutT*)dfk, (OutT*)dv, den, delta, p, dG, csum,
                       direct_dlg ? dlg : nullptr, H, L, F, D, gate, cps, KG, wg.per, wg.nx,
                       wg.nblk);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    return direct_dlg ? hipSuccess : launch_gate_grad(dG, csum, lg, dlg, B, H, L, gate, st);
  }
  auto launch_a = [&](auto tag) {
    constexpr auto kern = decltype(tag)::value;
    if (hipError_t e2 = ensure_lds<kern>(LDS_A); e2 != hipSuccess) return e2;
    hipLaunchKernelGGL(kern, dim3(wg.grid), dim3(B_THREADS), LDS_A, st, (const bf16*)fq,
                       (const bf16*)fk, (const bf16*)v, lg, (const bf16*)dy, (OutT*)dfq, den,
                       delta, p, fseg, H, L, F, D, gate, G, cps, M, KG, wg.per, wg.nx,
                       wg.nblk, flam);
    return hipGetLastError();
  };
  if (ext)
    e = launch_a(KernTag<gla_bwd_dq_kernel<FP, DP, OutT, VEC, true>>{});
  else if (CAN_FOLD && fold)
    e = launch_a(KernTag<gla_bwd_dq_kernel<FP, DP, OutT, VEC, false, CAN_FOLD>>{});
  else
    e = launch_a(KernTag<gla_bwd_dq_kernel<FP, DP, OutT, VEC, false>>{});
  if (e != hipSuccess) return e;
  float* rlam = rseg + (size_t)BH * G * SEG;
  if (G > 1) {
    auto ks = gla_bwd_state_kernel<FP, DP, VEC>;
    if ((e = ensure_lds<gla_bwd_state_kernel<FP, DP, VEC>>(LDS_S)) != hipSuccess) return e;
    hipLaunchKernelGGL(ks, dim3(BH * (G - 1)), dim3(256), LDS_S, st,
                       (const bf16*)fq, (const bf16*)dy, lg, (const float*)den,
                       (const float*)delta, rseg, rlam, H, L, F, D, gate, G, cps);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (!fold && (e = launch_gla_segment_scan(rseg, rlam, BH, G, SEG, true, st)) != hipSuccess)
      return e;
  }
  // more workgroups than CUs (one walk workgroup per CU): the dkv walk runs in
  // rounds, and takes its blocks in reverse so that its first round starts on
  // the rows the dq walk read last (measured on the unsegmented headline
  // before those ran fused: fwd+bwd -0.9 %; a one-round launch gains nothing
  // from the order)
  const int rev = wg.grid > device_geom().cus;
  auto launch_b = [&](auto tag) {
    constexpr auto kern = decltype(tag)::value;
    if (hipError_t e2 = ensure_lds<kern>(LDS_B); e2 != hipSuccess) return e2;
    hipLaunchKernelGGL(kern, dim3(wg.grid), dim3(B_THREADS), LDS_B, st, (const bf16*)fq,
                       (const bf16*)fk, (const bf16*)v, lg, (const bf16*)dy, (const float*)den,
                       (const float*)delta, (const float*)p, (OutT*)dfk, (OutT*)dv, dG, csum,
                       direct_dlg ? dlg : nullptr, (const float*)rseg, H, L, F, D, gate, G,
                       cps, M, KG, wg.per, wg.nx, wg.nblk, (const float*)rlam, rev);
    return hipGetLastError();
  };
  if (CAN_FOLD && fold)
    e = launch_b(KernTag<gla_bwd_dkv_kernel<FP, DP, OutT, VEC, CAN_FOLD>>{});
  else
    e = launch_b(KernTag<gla_bwd_dkv_kernel<FP, DP, OutT, VEC>>{});
  if (e != hipSuccess) return e;
  return direct_dlg ? hipSuccess : launch_gate_grad(dG, csum, lg, dlg, B, H, L, gate, st);
}

// ext_den / ext_delta: nullptr, or (one F tile of a split feature
// dimension) den and delta [BH, L] of the whole feature dimension
hipError_t launch_gla_bwd(const void* fq, const void* fk, const void* v, const float* lg,
                          const void* dy, void* dfq, void* dfk, void* dv, float* dlg,
                          bool grad_bf16, int B, int H, int L, int F, int D, int gate,
                          int KG, const float* fwd_ws, float* ws, const float* ext_den,
                          const float* ext_delta, hipStream_t st) {
  const int fp = gla_padded_dim(F), dp = gla_padded_dim(D);
  const bool vec = F % 8 == 0 && D % 8 == 0;
#define LZ_GLA_BWD_V(FPV, DPV, OUT, V)                                                          \
  launch_gla_bwd_t<FPV, DPV, OUT, V>(fq, fk, v, lg, dy, dfq, dfk, dv, dlg, B, H, L, F, D,      \
                                     gate, KG, fwd_ws, ws, ext_den, ext_delta, st)
#define LZ_GLA_BWD(FPV, DPV)                                                                    \
  if (fp == FPV && dp == DPV)                                                                   \
    return grad_bf16 ? (vec ? LZ_GLA_BWD_V(FPV, DPV, bf16, true)                                \
                            : LZ_GLA_BWD_V(FPV, DPV, bf16, false))                              \
                     : (vec ? LZ_GLA_BWD_V(FPV, DPV, float, true)                               \
                            : LZ_GLA_BWD_V(FPV, DPV, float, false));
  LZ_GLA_BWD(32, 32) LZ_GLA_BWD(32, 64) LZ_GLA_BWD(32, 128)
  LZ_GLA_BWD(64, 32) LZ_GLA_BWD(64, 64) LZ_GLA_BWD(64, 128)
  LZ_GLA_BWD(128, 32) LZ_GLA_BWD(128, 64) LZ_GLA_BWD(128, 128)
  LZ_GLA_BWD(256, 32) LZ_GLA_BWD(256, 64)
#undef LZ_GLA_BWD
#undef LZ_GLA_BWD_V
  return hipErrorInvalidValue;
}

}  // namespace lz
