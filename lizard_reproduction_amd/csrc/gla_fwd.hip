// Chunked gated linear attention, forward, for gfx950.
//
// Math (reference operator src/kernels/gla.py:259-263 with the chunk
// conventions of src/kernels/gla.py:19-101; dense form
// src/lizard_attention.py:20-31).  Per (b, h), tokens are cut into 64-token
// chunks.  Inside chunk n, lg_j is the inclusive sum of log_gamma over the
// chunk up to token j (so every absorbed factor exp(.) is <= 1):
//   Q~_i = fq_i e^{lg_i},  K~_t = bf16(fk_t e^{lg_end - lg_t})
//   a_it = bf16((fq_i . fk_t) e^{lg_i - lg_t}) for t <= i
//   o_i  = Q~_i bf16(S_n) + sum_t a_it v_t,  den_i = Q~_i . z_n + sum_t a_it
//   y_i  = o_i / max(den_i, FLT_MIN)
//   S_{n+1} = e^{lg_end} S_n + K~^T V,   z_{n+1} = e^{lg_end} z_n + sum_t K~_t
// The reference takes the same differences from a global cumsum G; the
// chunk-local sums here are the same numbers without the cancellation.  The
// reference also rounds Q~ to bf16 before both of its products; here the row
// scale e^{lg_i} multiplies the fp32 results of fq . S_n and fq . z_n instead
// (one rounding fewer, the same Q~ in numerator and denominator).
//
// Work decomposition.  A workgroup (4 waves) walks the chunks of one segment
// of one (b, h) in order, with the state S (F x D, fp32) in MFMA accumulator
// registers for the whole walk: no state goes to HBM, so HBM traffic is one
// read of fq, fk, v and the gate and one write of y.  When B*H alone cannot
// fill the GPU, the sequence is cut into G segments per (b, h):
//   1. gla_fwd_state_kernel: the state each segment (but the last) leaves
//      when it starts from zero, its z and its total log decay;
//   2. gla_segment_scan_kernel: exclusive scan over segments, giving the
//      state entering each segment (S_g = e^{Lambda_{g-1}} S_{g-1} + dS_{g-1});
//   3. gla_fwd_kernel: every segment walks its chunks from its entering state.
// With G = 1 only step 3 runs.
//
// Per chunk, inside gla_fwd_kernel:
//   * fq, fk, v sit in LDS as row-major [token][feature] tiles (16-byte
//     stores); the next chunk is already in flight into registers.
//   * phase 1: wave (kt, qt) computes one 32x32 tile of s^T = fk fq^T
//     (keys x queries), applies the causal decay in registers and publishes
//     the bf16 tile as ready-made MFMA operands (the tile of keys 32-63 x
//     queries 0-31 is causally zero: its wave takes most of the Q~.z work
//     instead, and phase 2 skips its fragments); Q~.z partials go to LDS; the
//     workgroup forms K~ = bf16(fk ks) once (16-byte row items, with their
//     column sums for z) and writes it over fk, which the scores no longer need.
//   * phase 2: a wave owns d-tiles of the output and the state: o^T = S^T fq^T
//     (S straight from its accumulators) scaled by qs, + V^T P^T, y = o / den;
//     then S <- e^{lg_end} S + K~^T V.  The operands that contract over tokens
//     (V^T, K~^T, V) come from LDS transpose reads of the row-major tiles.
//   * the prefetched chunk is written to LDS, the gate scan of the next chunk
//     runs on wave 0, and z is updated.
#include "gla_common.hpp"

namespace lz {

template <int FP, int DP>
struct GlaFwd {
  static constexpr int C = GLA_C;
  static constexpr int PF = lds_pitch(FP), PD = lds_pitch(DP);   // LDS row pitches
  static constexpr int NFT = FP / 32, NDT = DP / 32;
  static constexpr int NLF = C * FP / 8 / 256;        // 16-byte loads per thread, fq or fk
  static constexpr int NLD = C * DP / 8 / 256;        // 16-byte loads per thread, v
  static constexpr int OFF_FQ = 0;
  static constexpr int OFF_FK = OFF_FQ + C * PF * 2;
  static constexpr int OFF_V = OFF_FK + C * PF * 2;
  static constexpr int OFF_PF = OFF_V + C * PD * 2;      // [2 qt][4 kb][64 lanes] bf16x8
  static constexpr int OFF_RS = OFF_PF + 2 * 4 * 64 * 16; // [2 kt][64] row sums of a
  static constexpr int OFF_QZ = OFF_RS + 2 * 64 * 4;      // [4 waves][64] Q~.z partials
  static constexpr int OFF_LG = OFF_QZ + 4 * 64 * 4;      // [64] chunk-local lg
  static constexpr int OFF_QS = OFF_LG + 64 * 4;          // [64] e^{lg}
  static constexpr int OFF_KS = OFF_QS + 64 * 4;          // [64] e^{lg_end - lg}
  static constexpr int OFF_Z = OFF_KS + 64 * 4;           // [FP] z
  static constexpr int OFF_ZP = OFF_Z + FP * 4;           // 2048 partial sums of K~
  static constexpr int OFF_R = OFF_ZP + 2048 * 4;         // e^{lg_end}, lg_end
  static constexpr int BYTES = OFF_R + 16;
  static constexpr int SEG = SegRec<FP, DP>::SIZE;
  // two workgroups per CU up to F = 128 (the launch bounds ask for it), one beyond
  static_assert(BYTES <= (FP >= 256 ? 160 : 80) * 1024, "LDS budget");
};

// ----------------------------------------------------------------------------
// fused forward walk over the chunks of one segment
// ----------------------------------------------------------------------------
// RAW (one F tile of a split feature dimension): instead of y, the walk writes
// the unnormalised numerator o (fp32 [BH, L, D] at raw_num) and denominator
// (fp32 [BH, L] at raw_den), which the caller sums over the F tiles.
template <int FP, int DP, bool VEC, bool RAW, bool FOLD = false, bool NTL = false>
__global__ __launch_bounds__(256, FP >= 256 ? 1 : 2) void gla_fwd_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, bf16* __restrict__ y,
    const float* __restrict__ seg_state, float* __restrict__ final_state, int H, int L, int F,
    int D, int gate, int G, int cps, int M, int KG, float* __restrict__ raw_num,
    float* __restrict__ raw_den, int xper, int nxcd, int nblk, const float* __restrict__ seg_lam) {
  using Cfg = GlaFwd<FP, DP>;
  constexpr int C = Cfg::C, PF = Cfg::PF, PD = Cfg::PD;
  constexpr int NFT = Cfg::NFT, NDT = Cfg::NDT;
  using RD = Roles<NDT>;   // wave -> owned d-tiles (state and output) x output q-tiles
  // NTL: the chunk loads are nontemporal (one segment, no shared kv heads:
  // nothing reads these rows again during the walk)
  constexpr int AUX = NTL ? LOAD_NT : 0;
  constexpr int NDW = RD::TILES, NQW = RD::HALVES;
  extern __shared__ __align__(16) char smem[];
  bf16* fq_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQ);
  bf16* fk_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FK);
  bf16* v_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_V);
  bf16x8* pfrag = reinterpret_cast<bf16x8*>(smem + Cfg::OFF_PF);
  float* rs = reinterpret_cast<float*>(smem + Cfg::OFF_RS);
  float* qz = reinterpret_cast<float*>(smem + Cfg::OFF_QZ);
  float* lgs = reinterpret_cast<float*>(smem + Cfg::OFF_LG);
  float* qs = reinterpret_cast<float*>(smem + Cfg::OFF_QS);
  float* ks = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  float* zs = reinterpret_cast<float*>(smem + Cfg::OFF_Z);
  float* zp = reinterpret_cast<float*>(smem + Cfg::OFF_ZP);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  // a workgroup walks M consecutive segments seg .. seg + M - 1 from the
  // state entering the first; logical block b = bh nwg + segment / M
  const int nwg = G / M;
  int blk;
  if (!walk_block(xper, nxcd, nblk, blk)) return;
  const int bh = blk / nwg, seg = (blk % nwg) * M;
  const int NT = (L + C - 1) / C;
  const int n0 = seg * cps, n1 = min(NT, n0 + M * cps);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const bool vecF = VEC || (F & 7) == 0, vecD = VEC || (D & 7) == 0;
  // fk and v belong to the kv head of this query head: KG query heads share one
  const bf16* fqb = fq + (size_t)bh * L * F;
  const bf16* fkb = fk + (size_t)(bh / KG) * L * F;
  const bf16* vb = v + (size_t)(bh / KG) * L * D;
  const rsrc_t yr = make_rsrc(y + (size_t)bh * L * D, (size_t)L * D * 2);
  const float* lgb = log_gamma + (size_t)((gate & GATE_PER_HEAD) ? bh : bh / H) * L;
  // the state entering segment seg: its scanned record, or (FOLD) the local
  // records of segments 0 .. seg - 1 folded here (their total log decays at
  // seg_lam)
  const int own = seg_owner_uniform(bh, KG, gate);
  const float* st =
      G > 1 ? seg_state + ((size_t)own * G + (FOLD ? 0 : seg)) * Cfg::SEG : nullptr;

  const bool active = RD::active(wave);
  auto dtile = [&](int i) { return RD::tile(wave, i); };
  auto qtile = [&](int j) { return RD::half(wave, j); };

  f32x16 S[NDW][NFT];
  if constexpr (FOLD) {   // folded in LDS, before the first chunk is staged there
    static_assert(Cfg::SEG * 4 <= Cfg::BYTES, "a folded record fits the chunk's LDS");
    float* fold_l = reinterpret_cast<float*>(smem);
    if (seg > 0)
      fold_records<256, Cfg::SEG, 64>(fold_l, st, seg_lam + (size_t)own * G, 0, 1, seg);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NDW; ++i)
#pragma unroll
      for (int ft = 0; ft < NFT; ++ft) {
        S[i][ft] = zero16();
        if (seg > 0 && active) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            S[i][ft][r] = fold_l[(ft * 32 + acc_row(r, h)) * DP + dtile(i) * 32 + col];
        }
      }
    static_assert(FP <= 256, "one z element per thread");
    const float zv = seg > 0 && tid < FP ? fold_l[FP * DP + tid] : 0.f;
    __syncthreads();   // read before the LDS is reused
    if (tid < FP) zs[tid] = zv;
  } else {
#pragma unroll
    for (int i = 0; i < NDW; ++i)
#pragma unroll
      for (int ft = 0; ft < NFT; ++ft) {
        S[i][ft] = zero16();
        if (st && active) {
#pragma unroll
          for (int r = 0; r < 16; ++r)
            S[i][ft][r] = st[(ft * 32 + acc_row(r, h)) * DP + dtile(i) * 32 + col];
        }
      }
    for (int f = tid; f < FP; f += 256) zs[f] = st ? st[FP * DP + f] : 0.f;
  }

  uint4 rq[Cfg::NLF], rk[Cfg::NLF], rv[Cfg::NLD];
  float rg;
  load_chunk<FP, Cfg::NLF, AUX>(rq, fqb, n0 * C, L, F, vecF);
  load_chunk<FP, Cfg::NLF, AUX>(rk, fkb, n0 * C, L, F, vecF);
  load_chunk<DP, Cfg::NLD, AUX>(rv, vb, n0 * C, L, D, vecD);
  rg = gate_at(lgb, n0 * C + lane, L);
  store_chunk<FP>(rq, fq_l, PF);
  store_chunk<FP>(rk, fk_l, PF);
  store_chunk<DP>(rv, v_l, PD);
  if (wave == 0) gate_scan(rg, lane, lgs, qs, ks, rdec, gate, n0 * C + lane < L);
  __syncthreads();

  for (int n = n0; n < n1; ++n) {
    const int t0 = n * C;
    const bool more = n + 1 < n1;
    if (more) {   // next chunk in flight while this one computes
      load_chunk<FP, Cfg::NLF, AUX>(rq, fqb, t0 + C, L, F, vecF);
      load_chunk<FP, Cfg::NLF, AUX>(rk, fkb, t0 + C, L, F, vecF);
      load_chunk<DP, Cfg::NLD, AUX>(rv, vb, t0 + C, L, D, vecD);
      rg = gate_at(lgb, t0 + C + lane, L);
    }
    __builtin_amdgcn_s_setprio(0);
    // ---- phase 1: scores -> P fragments and row sums; fq.z; K~ rows --------
    uint4 kti[RowItems<FP>::N];   // this thread's rows of K~ = bf16(fk * ks)
    {
      const int kt = wave >> 1, qt = wave & 1;
      const int qi = qt * 32 + col;
      if (kt == 1 && qt == 0) {
        // keys 32-63 x queries 0-31: causally zero (phase 2 skips its fragments)
        if (h == 0) rs[64 + qi] = 0.f;
      } else {
        f32x16 s = zero16();
#pragma unroll
        for (int kb = 0; kb < FP / 16; ++kb)
          s = mfma(row_operand(fk_l, PF, kt * 32 + col, 16 * kb, h),
                   row_operand(fq_l, PF, qi, 16 * kb, h), s);
        bf16x8 p[2];
        float rsum = decay_tile(s, lgs, kt, qi, h, p);
        rsum += xhalf(rsum);
        pfrag[(qt * 4 + kt * 2 + 0) * 64 + lane] = p[0];
        pfrag[(qt * 4 + kt * 2 + 1) * 64 + lane] = p[1];
        if (h == 0) rs[kt * 64 + qi] = rsum;
      }

      // qs (fq . z), query = lane, over 8-feature groups: wave 2 (no score
      // tile) takes 5/8 of the groups, waves 0, 1, 3 a third of the rest each
      constexpr int NG = FP / 8, G2 = NG * 5 / 8, GR = NG - G2;
      const int wi = wave == 3 ? 2 : wave;
      const int g0 = wave == 2 ? 0 : G2 + wi * GR / 3;
      const int g1 = wave == 2 ? G2 : G2 + (wi + 1) * GR / 3;
      float acc = 0.f;
#pragma unroll 2
      for (int g = g0; g < g1; ++g) {
        const bf16x8 x = *reinterpret_cast<const bf16x8*>(fq_l + lane * PF + 8 * g);
        const f32x4 z0 = *reinterpret_cast<const f32x4*>(zs + 8 * g);
        const f32x4 z1 = *reinterpret_cast<const f32x4*>(zs + 8 * g + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += to_f32(x[e]) * z0[e];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += to_f32(x[4 + e]) * z1[e];
      }
      qz[wave * 64 + lane] = acc * qs[lane];
      scale_rows<FP>(fk_l, PF, ks, kti, zp);
    }
    __syncthreads();
    store_rows<FP>(kti, fk_l, PF);   // fk_l holds K~ from here to the end of the chunk
    __syncthreads();
    // ---- phase 2: outputs and state update ----------------------------------
    const float r_n = rdec[0];
    if (active) {
#pragma unroll
      for (int i = 0; i < NDW; ++i) {
        const int dt = dtile(i);
        bf16x8 vop[4];   // V^T rows of this d-tile (A of V^T P^T) == V columns (B of K~^T V)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) vop[kb] = tr_operand(v_l, PD, 16 * kb, dt * 32, lane);
#pragma unroll
        for (int j = 0; j < NQW; ++j) {
          const int qt = qtile(j);
          const int qi = qt * 32 + col;
          // o^T = qs (S^T fq^T) + V^T P^T: the row scale of Q~ = fq qs is applied to the
          // fp32 product (den uses the same unrounded Q~, so L = 1 still gives y = v)
          // LDS operands are read a group ahead of the products that use them
          constexpr int KB = FP / 16, KG4 = KB < 4 ? KB : 4;
          f32x16 o = zero16();
#pragma unroll
          for (int k4 = 0; k4 < KB / KG4; ++k4) {
            bf16x8 fop[KG4];
#pragma unroll
            for (int u = 0; u < KG4; ++u)
              fop[u] = row_operand_acc(fq_l, PF, qi, 16 * (KG4 * k4 + u), h);
#pragma unroll
            for (int u = 0; u < KG4; ++u) {
              const int kb = KG4 * k4 + u;
              o = mfma(acc_operand(S[i][kb >> 1], kb & 1), fop[u], o);
            }
          }
          bf16x8 pop[4];
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)   // queries 0-31 have no keys in blocks 2, 3
            if (qt == 1 || kb < 2) pop[kb] = pfrag[(qt * 4 + kb) * 64 + lane];
          const float qsv = qs[qi];
          const float d0 = rs[qi], d1 = rs[64 + qi], d2 = qz[qi], d3 = qz[64 + qi];
          const float d4 = qz[128 + qi], d5 = qz[192 + qi];
#pragma unroll
          for (int r = 0; r < 16; ++r) o[r] *= qsv;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
            if (qt == 1 || kb < 2) o = mfma(vop[kb], pop[kb], o);
          const float den = d0 + d1 + d2 + d3 + d4 + d5;
          if constexpr (RAW) {
            store_acc_row<float>(raw_num + (size_t)bh * L * D, t0 + qi, dt * 32, L, D, vecD, o,
                                 1.f, h);
            if (dt == 0 && h == 0 && t0 + qi < L) raw_den[(size_t)bh * L + t0 + qi] = den;
          } else {
            store_acc_row_bf16(yr, t0 + qi, dt * 32, D, vecD, o, recip_den(den), h);
          }
        }
#pragma unroll
        for (int ft = 0; ft < NFT; ++ft) {
          // the four K~^T operands of this f-tile are read before its products
          bf16x8 kop[4];
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) kop[kb] = tr_operand(fk_l, PF, 16 * kb, ft * 32, lane);
#pragma unroll
          for (int r = 0; r < 16; ++r) S[i][ft][r] *= r_n;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb) S[i][ft] = mfma(kop[kb], vop[kb], S[i][ft]);
          __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);   // the 8 transpose reads
          __builtin_amdgcn_sched_group_barrier(0x002, 16, 0);  // the decay of S
          __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);   // the 4 products
        }
      }
    }
    __syncthreads();
    // ---- next chunk into LDS; z update ----------------------------------------
    // the staging of the next chunk and the issue of the loads after it run at
    // raised wave priority: the other workgroup on the CU is then usually in its
    // compute phases, and the chunk's loads leave as early as they can
    __builtin_amdgcn_s_setprio(1);
    if (more) {
      store_chunk<FP>(rq, fq_l, PF);
      store_chunk<FP>(rk, fk_l, PF);
      store_chunk<DP>(rv, v_l, PD);
      if (wave == 0) gate_scan(rg, lane, lgs, qs, ks, rdec, gate, t0 + C + lane < L);
    }
    if (tid < FP) zs[tid] = zs[tid] * r_n + sum_parts<FP>(zp, tid);
    __syncthreads();
  }

  // the state after the whole sequence, [F][D] fp32 then z [F], for decoding
  if (final_state && seg + M == G) {
    float* fs = final_state + (size_t)bh * ((size_t)F * D + F);
    if (active && RD::primary(wave)) {
#pragma unroll
      for (int i = 0; i < NDW; ++i) {
        const int d = dtile(i) * 32 + col;
#pragma unroll
        for (int ft = 0; ft < NFT; ++ft)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int f = ft * 32 + acc_row(r, h);
            if (f < F && d < D) fs[(size_t)f * D + d] = S[i][ft][r];
          }
      }
    }
    for (int f = tid; f < F; f += 256) fs[(size_t)F * D + f] = zs[f];
  }
}

// ----------------------------------------------------------------------------
// F = 256: the same walk with eight waves per workgroup.  At F = 256 a chunk's
// tiles leave room for one workgroup per CU, so the four-wave walk above runs
// one wave per SIMD and its two waves per d-tile both carry (and update) that
// tile's whole state.  Here 512 threads share the chunk, two waves per SIMD:
//   * every (f-tile, d-tile) tile of S lives in exactly one wave's
//     accumulators (tile t = wave + 8 i), and after each update the waves
//     publish bf16 S^T [d][f] to LDS, where the output products read it: the
//     same bf16(S) operands, in the same k order, as the register form above;
//   * phase 1: waves 0, 1, 3 compute the three score tiles that are not
//     causally zero; wave 2 takes 5/8 of the Q~.z feature groups, waves 4-7
//     the rest and K~ = bf16(fk ks) with its column sums;
//   * phase 2: waves 4-7 (4 - 4 + 2 NDT of them) compute the outputs of one
//     (d-tile, query half) each; all waves update their state tiles;
//   * then the waves publish S^T, stage the prefetched chunk, scan the next
//     gate and update z.
// ----------------------------------------------------------------------------
constexpr int WIDE_THREADS = 512;

template <int DP>
struct GlaFwdWide {
  static constexpr int FP = 256, C = GLA_C;
  static constexpr int PF = lds_pitch(FP), PD = lds_pitch(DP);
  static constexpr int NFT = FP / 32, NDT = DP / 32;
  static constexpr int S_OWN = (NFT * NDT + 7) / 8;          // state tiles per wave
  static constexpr int NLF = C * FP / 8 / WIDE_THREADS;       // 16-byte items per thread, fq or fk
  static constexpr int NLD = (C * DP / 8 + WIDE_THREADS - 1) / WIDE_THREADS;
  static constexpr int OFF_FQ = 0;
  static constexpr int OFF_FK = OFF_FQ + C * PF * 2;
  static constexpr int OFF_V = OFF_FK + C * PF * 2;
  static constexpr int OFF_ST = OFF_V + C * PD * 2;           // bf16 S^T [DP][PF]
  static constexpr int OFF_PF = OFF_ST + DP * PF * 2;         // [2 qt][4 kb][64 lanes] bf16x8
  static constexpr int OFF_RS = OFF_PF + 2 * 4 * 64 * 16;     // [2 kt][64] row sums of a
  static constexpr int OFF_QZ = OFF_RS + 2 * 64 * 4;          // [8 waves][64] Q~.z partials
  static constexpr int OFF_LG = OFF_QZ + 8 * 64 * 4;
  static constexpr int OFF_QS = OFF_LG + 64 * 4;
  static constexpr int OFF_KS = OFF_QS + 64 * 4;
  static constexpr int OFF_Z = OFF_KS + 64 * 4;
  static constexpr int OFF_ZP = OFF_Z + FP * 4;               // K~ column partial sums
  static constexpr int OFF_R = OFF_ZP + RowItems<FP>::PARTS * FP * 4;
  static constexpr int BYTES = OFF_R + 16;
  static_assert(BYTES <= 160 * 1024, "LDS budget");
  // PHI: softmax statistics of q W^T per (token tile, 32-feature tile, token),
  // and W [128][PW] bf16 (head_dim 64)
  static constexpr int PW = lds_pitch(64);
  static constexpr int OFF_PS = BYTES;
  static constexpr int OFF_W = OFF_PS + 2 * 4 * 32 * 16;
  static constexpr int PHI_BYTES = OFF_W + 128 * PW * 2;
  static_assert(PHI_BYTES <= 160 * 1024, "LDS budget");
};

// rows [t0, t0+64) of a [L x ncols] bf16 matrix by the 512 threads (item
// idx = tid + 512 i: row idx / (KP/8), 8 columns), and their LDS stores
template <int KP, int N>
__device__ __forceinline__ void load_chunk512(uint4 (&reg)[N], const bf16* __restrict__ base,
                                              int t0, int L, int ncols, bool vec) {
  load_items<KP, WIDE_THREADS, N, GLA_C * KP / 8>(reg, base, t0, L, ncols, vec);
}

template <int KP, int N>
__device__ __forceinline__ void store_chunk512(const uint4 (&reg)[N], bf16* tile, int pitch) {
  constexpr int K8 = KP / 8, ITEMS = GLA_C * K8;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int idx = threadIdx.x + WIDE_THREADS * i;
    if (ITEMS % WIDE_THREADS == 0 || idx < ITEMS)
      *reinterpret_cast<uint4*>(tile + (idx / K8) * pitch + (idx % K8) * 8) = reg[i];
  }
}

// PHI: fq is not read.  The walk forms it from the q rows of the projection
// output (qrow, [B, L, H, 64] bf16) and the feature weights (wphi, [128][64]
// bf16) chunk by chunk: fq = [softmax(q W^T), softmax(-q W^T)] (the Hedgehog
// map, src/lizard_attention.py:9-11, F = 256), as the layer prologue does:
// the same bf16 MFMA product (A = W rows, B = q rows, k over head_dim in the
// same order, so x W^T is bitwise the prologue's), fp32 softmax with the row
// maximum subtracted, bf16 result.  Wave w forms 32-feature tile w >> 1 of
// 32-token tile w & 1; the statistics of a token's four tiles meet in LDS
// (written in phase 2, read in the tail, where the chunk is staged: no barrier
// of its own), combined as max M and sum of s_j e^{m_j - M}.
template <int DP, bool VEC, bool RAW, bool PHI, bool FOLD = false>
__global__ __launch_bounds__(WIDE_THREADS, 1) void gla_fwd_wide_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, bf16* __restrict__ y,
    const float* __restrict__ seg_state, float* __restrict__ final_state, int H, int L, int F,
    int D, int gate, int G, int cps, int M, int KG, float* __restrict__ raw_num,
    float* __restrict__ raw_den, int xper, int nxcd, int nblk, const bf16* __restrict__ qrow,
    const bf16* __restrict__ wphi, const float* __restrict__ seg_lam) {
  static_assert(!(PHI && RAW), "the feature map is formed for whole-F walks only");
  using Cfg = GlaFwdWide<DP>;
  constexpr int FP = Cfg::FP, C = Cfg::C, PF = Cfg::PF, PD = Cfg::PD;
  constexpr int NFT = Cfg::NFT, NDT = Cfg::NDT, S_OWN = Cfg::S_OWN;
  extern __shared__ __align__(16) char smem[];
  bf16* fq_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FQ);
  bf16* fk_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FK);
  bf16* v_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_V);
  bf16* st_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_ST);
  bf16x8* pfrag = reinterpret_cast<bf16x8*>(smem + Cfg::OFF_PF);
  float* rs = reinterpret_cast<float*>(smem + Cfg::OFF_RS);
  float* qz = reinterpret_cast<float*>(smem + Cfg::OFF_QZ);
  float* lgs = reinterpret_cast<float*>(smem + Cfg::OFF_LG);
  float* qs = reinterpret_cast<float*>(smem + Cfg::OFF_QS);
  float* ks = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  float* zs = reinterpret_cast<float*>(smem + Cfg::OFF_Z);
  float* zp = reinterpret_cast<float*>(smem + Cfg::OFF_ZP);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  const int nwg = G / M;
  int blk;
  if (!walk_block(xper, nxcd, nblk, blk)) return;
  const int bh = blk / nwg, seg = (blk % nwg) * M;
  const int NT = (L + C - 1) / C;
  const int n0 = seg * cps, n1 = min(NT, n0 + M * cps);
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const bool vecF = VEC || (F & 7) == 0, vecD = VEC || (D & 7) == 0;
  const bf16* fqb = fq + (size_t)bh * L * F;
  const bf16* fkb = fk + (size_t)(bh / KG) * L * F;   // fk, v: the kv head of this query head
  const bf16* vb = v + (size_t)(bh / KG) * L * D;
  const rsrc_t yr = make_rsrc(y + (size_t)bh * L * D, (size_t)L * D * 2);
  const float* lgb = log_gamma + (size_t)((gate & GATE_PER_HEAD) ? bh : bh / H) * L;
  // the state entering segment seg: its scanned record, or (FOLD) the local
  // records of segments 0 .. seg - 1 folded here (their total log decays at
  // seg_lam)
  constexpr int SEG = SegRec<FP, DP>::SIZE;
  const int own = seg_owner_uniform(bh, KG, gate);
  const float* st = G > 1 ? seg_state + ((size_t)own * G + (FOLD ? 0 : seg)) * SEG : nullptr;

  // state tile i of this wave: t = wave + 8 i -> f-tile t % NFT, d-tile t / NFT
  f32x16 S[S_OWN];
  if constexpr (FOLD) {   // folded in LDS, before the first chunk is staged there
    static_assert(SEG * 4 <= Cfg::BYTES, "a folded record fits the chunk's LDS");
    float* fold_l = reinterpret_cast<float*>(smem);
    if (seg > 0)
      fold_records<WIDE_THREADS, SEG, 160>(fold_l, st, seg_lam + (size_t)own * G, 0, 1, seg);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < S_OWN; ++i) {
      S[i] = zero16();
      const int t = wave + 8 * i, ft = t % NFT, dt = t / NFT;
      if (seg > 0 && t < NFT * NDT) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          S[i][r] = fold_l[(ft * 32 + acc_row(r, h)) * DP + dt * 32 + col];
      }
    }
    static_assert(FP <= WIDE_THREADS, "one z element per thread");
    const float zv = seg > 0 && tid < FP ? fold_l[FP * DP + tid] : 0.f;
    __syncthreads();   // read before the LDS is reused
    if (tid < FP) zs[tid] = zv;
  } else {
#pragma unroll
    for (int i = 0; i < S_OWN; ++i) {
      S[i] = zero16();
      const int t = wave + 8 * i, ft = t % NFT, dt = t / NFT;
      if (st && t < NFT * NDT) {
#pragma unroll
        for (int r = 0; r < 16; ++r) S[i][r] = st[(ft * 32 + acc_row(r, h)) * DP + dt * 32 + col];
      }
    }
    for (int f = tid; f < FP; f += WIDE_THREADS) zs[f] = st ? st[FP * DP + f] : 0.f;
  }
  // bf16 S^T [d][f] (4 consecutive f per store), read by the output products
  auto publish = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < S_OWN; ++i) {
      const int t = wave + 8 * i;
      if (t < NFT * NDT) {
        const int ft = t % NFT, d = (t / NFT) * 32 + col;
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          bf16x4 o;
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = to_bf16(S[i][4 * g4 + e]);
          *reinterpret_cast<bf16x4*>(st_l + d * PF + ft * 32 + 8 * g4 + 4 * h) = o;
        }
      }
    }
  };

  // ---- PHI: the feature map of q, formed per chunk -------------------------
  constexpr int PHD = 64, PHK = PHD / 16;   // head_dim of q and W; MFMA k-steps
  const int ptt = wave & 1, pft = wave >> 1;
  uint4 px[PHK];     // the next chunk's q rows of token tile ptt (B operand)
  f32x16 pacc;       // q W^T tile: features 32 pft + acc_row (registers) x tokens (lanes)
  f32x4* pst = reinterpret_cast<f32x4*>(smem + Cfg::OFF_PS);
  bf16* w_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_W);   // W, for the whole walk
  // q rows of this (b, h): token t at (t H) PHD elements past its first row
  const rsrc_t qrs = make_rsrc(
      PHI ? qrow + ((size_t)(bh / H) * L * H + (size_t)(bh % H)) * PHD : nullptr,
      PHI ? ((size_t)(L - 1) * H + 1) * PHD * 2 : 0);
  auto phi_load = [&](int t) __attribute__((always_inline)) {   // chunk starting at t
    const int row = t + 32 * ptt + col;
#pragma unroll
    for (int kb = 0; kb < PHK; ++kb)
      px[kb] = bload16(qrs, row < L ? (uint32_t)((row * H * PHD + 16 * kb + 8 * h) * 2) : OOB);
  };
  // this wave's tile of q W^T and its per-token statistics (max and sum of
  // e^{x - max} over the tile's 32 features, both signs) into LDS
  auto phi_partial = [&]() __attribute__((always_inline)) {
    pacc = zero16();
#pragma unroll
    for (int kb = 0; kb < PHK; ++kb)
      pacc = mfma(row_operand(w_l, Cfg::PW, 32 * pft + col, 16 * kb, h),
                  __builtin_bit_cast(bf16x8, px[kb]), pacc);
    float mp = pacc[0], mn = -pacc[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) {
      mp = fmaxf(mp, pacc[r]);
      mn = fmaxf(mn, -pacc[r]);
    }
    mp = fmaxf(mp, xhalf(mp));
    mn = fmaxf(mn, xhalf(mn));
    // e^{x - m} as exp2 of one FMA
    const float cp = -mp * LOG2E, cn = -mn * LOG2E;
    float sp = 0.f, sn = 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sp += __builtin_amdgcn_exp2f(fmaf(pacc[r], LOG2E, cp));
      sn += __builtin_amdgcn_exp2f(fmaf(pacc[r], -LOG2E, cn));
    }
    sp += xhalf(sp);
    sn += xhalf(sn);
    if (h == 0) pst[(ptt * 4 + pft) * 32 + col] = f32x4{mp, sp, mn, sn};
  };
  // after a barrier: the token's statistics over all 128 features, and this
  // wave's 32 features of both halves of its fq row into fq_l (zero past L)
  auto phi_write = [&](int t) __attribute__((always_inline)) {
    f32x4 g[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) g[j] = pst[(ptt * 4 + j) * 32 + col];
    const float Mp = fmaxf(fmaxf(g[0][0], g[1][0]), fmaxf(g[2][0], g[3][0]));
    const float Mn = fmaxf(fmaxf(g[0][2], g[1][2]), fmaxf(g[2][2], g[3][2]));
    float Sp = 0.f, Sn = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      Sp += g[j][1] * fexp(g[j][0] - Mp);
      Sn += g[j][3] * fexp(g[j][2] - Mn);
    }
    // e^{x - M} / S = exp2(x log2e - (M log2e + log2 S)): one FMA and exp2
    const float op_ = -(Mp * LOG2E + __builtin_amdgcn_logf(Sp));
    const float on_ = -(Mn * LOG2E + __builtin_amdgcn_logf(Sn));
    const int tok = 32 * ptt + col;
    const bool live = t + tok < L;
    bf16* row = fq_l + tok * PF + 32 * pft;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      bf16x4 op, on;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = pacc[4 * q4 + e];
        op[e] = to_bf16(live ? __builtin_amdgcn_exp2f(fmaf(x, LOG2E, op_)) : 0.f);
        on[e] = to_bf16(live ? __builtin_amdgcn_exp2f(fmaf(x, -LOG2E, on_)) : 0.f);
      }
      *reinterpret_cast<bf16x4*>(row + 8 * q4 + 4 * h) = op;
      *reinterpret_cast<bf16x4*>(row + 128 + 8 * q4 + 4 * h) = on;
    }
  };

  uint4 rq[Cfg::NLF], rk[Cfg::NLF], rv[Cfg::NLD];
  float rg;
  if constexpr (PHI)
    phi_load(n0 * C);
  else
    load_chunk512<FP>(rq, fqb, n0 * C, L, F, vecF);
  load_chunk512<FP>(rk, fkb, n0 * C, L, F, vecF);
  load_chunk512<DP>(rv, vb, n0 * C, L, D, vecD);
  rg = gate_at(lgb, n0 * C + lane, L);

  if constexpr (PHI) {
    for (int i = tid; i < 128 * PHD / 8; i += WIDE_THREADS)
      *reinterpret_cast<uint4*>(w_l + (i / (PHD / 8)) * Cfg::PW + 8 * (i % (PHD / 8))) =
          reinterpret_cast<const uint4*>(wphi)[i];
  }
  if constexpr (!PHI) store_chunk512<FP>(rq, fq_l, PF);
  store_chunk512<FP>(rk, fk_l, PF);
  store_chunk512<DP>(rv, v_l, PD);
  if (wave == 0) gate_scan(rg, lane, lgs, qs, ks, rdec, gate, n0 * C + lane < L);
  publish();
  if constexpr (PHI) {
    __syncthreads();   // W in LDS
    phi_partial();
    __syncthreads();
    phi_write(n0 * C);
  }
  __syncthreads();

  // phase-1 roles: score tile (kt, qt) of waves 0, 1, 3; Q~.z groups of wave
  // 2 (5/8 of them) and waves 4-7 (the rest, a quarter each)
  constexpr int NG = FP / 8, G2 = NG * 5 / 8, GR = NG - G2;
  const int g0 = wave == 2 ? 0 : G2 + (wave - 4) * GR / 4;
  const int g1 = wave == 2 ? G2 : G2 + (wave - 3) * GR / 4;
  const bool qz_wave = wave == 2 || wave >= 4;
  for (int n = n0; n < n1; ++n) {
    const int t0 = n * C;
    const bool more = n + 1 < n1;
    if (more) {   // next chunk in flight while this one computes
      if constexpr (PHI)
        phi_load(t0 + C);
      else
        load_chunk512<FP>(rq, fqb, t0 + C, L, F, vecF);
      load_chunk512<FP>(rk, fkb, t0 + C, L, F, vecF);
      load_chunk512<DP>(rv, vb, t0 + C, L, D, vecD);
      rg = gate_at(lgb, t0 + C + lane, L);
    }
    // ---- phase 1 ------------------------------------------------------------
    uint4 kti[RowItems<FP>::N];   // waves 4-7: their rows of K~ = bf16(fk * ks)
    if (wave < 4 && wave != 2) {
      const int kt = wave >> 1, qt = wave & 1;
      const int qi = qt * 32 + col;
      f32x16 s = zero16();
#pragma unroll
      for (int kb = 0; kb < FP / 16; ++kb)
        s = mfma(row_operand(fk_l, PF, kt * 32 + col, 16 * kb, h),
                 row_operand(fq_l, PF, qi, 16 * kb, h), s);
      bf16x8 p[2];
      float rsum = decay_tile(s, lgs, kt, qi, h, p);
      rsum += xhalf(rsum);
      pfrag[(qt * 4 + kt * 2 + 0) * 64 + lane] = p[0];
      pfrag[(qt * 4 + kt * 2 + 1) * 64 + lane] = p[1];
      if (h == 0) rs[kt * 64 + qi] = rsum;
    }
    if (wave == 2 && h == 0) rs[64 + col] = 0.f;   // keys 32-63 x queries 0-31: zero
    if (qz_wave) {
      float acc = 0.f;
#pragma unroll 2
      for (int g = g0; g < g1; ++g) {
        const bf16x8 x = *reinterpret_cast<const bf16x8*>(fq_l + lane * PF + 8 * g);
        const f32x4 z0 = *reinterpret_cast<const f32x4*>(zs + 8 * g);
        const f32x4 z1 = *reinterpret_cast<const f32x4*>(zs + 8 * g + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += to_f32(x[e]) * z0[e];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc += to_f32(x[4 + e]) * z1[e];
      }
      qz[wave * 64 + lane] = acc * qs[lane];
    }
    if (wave >= 4) scale_rows_t<FP>(fk_l, PF, ks, kti, zp, tid - 256);
    __syncthreads();
    if (wave >= 4) store_rows_t<FP>(kti, fk_l, PF, tid - 256);   // fk_l holds K~ from here
    __syncthreads();
    // ---- phase 2: outputs (waves 4 .. 3 + 2 NDT), state update (all) ---------
    // PHI: the next chunk's q W^T tile and its statistics, waves 0-3 first
    // (their phase 2 is the state update only), waves 4-7 after their outputs
    if constexpr (PHI) {
      if (more && wave < 4) phi_partial();
    }
    const float r_n = rdec[0];
    if (wave >= 4 && wave < 4 + 2 * NDT) {
      const int dt = (wave - 4) >> 1, qt = (wave - 4) & 1;
      const int qi = qt * 32 + col;
      f32x16 o = zero16();
#pragma unroll
      for (int kb = 0; kb < FP / 16; ++kb)
        o = mfma(row_operand(st_l, PF, dt * 32 + col, 16 * kb, h),
                 row_operand(fq_l, PF, qi, 16 * kb, h), o);
      const float qsv = qs[qi];
#pragma unroll
      for (int r = 0; r < 16; ++r) o[r] *= qsv;
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)   // queries 0-31 have no keys in blocks 2, 3
        if (qt == 1 || kb < 2)
          o = mfma(tr_operand(v_l, PD, 16 * kb, dt * 32, lane), pfrag[(qt * 4 + kb) * 64 + lane], o);
      float den = rs[qi] + rs[64 + qi] + qz[2 * 64 + qi];
#pragma unroll
      for (int w = 4; w < 8; ++w) den += qz[w * 64 + qi];
      if constexpr (RAW) {   // as in gla_fwd_kernel
        store_acc_row<float>(raw_num + (size_t)bh * L * D, t0 + qi, dt * 32, L, D, vecD, o, 1.f,
                             h);
        if (dt == 0 && h == 0 && t0 + qi < L) raw_den[(size_t)bh * L + t0 + qi] = den;
      } else {
        store_acc_row_bf16(yr, t0 + qi, dt * 32, D, vecD, o, recip_den(den), h);
      }
    }
#pragma unroll
    for (int i = 0; i < S_OWN; ++i) {
      const int t = wave + 8 * i, ft = t % NFT, dt = t / NFT;
      if (t < NFT * NDT) {
#pragma unroll
        for (int r = 0; r < 16; ++r) S[i][r] *= r_n;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
          S[i] = mfma(tr_operand(fk_l, PF, 16 * kb, ft * 32, lane),
                      tr_operand(v_l, PD, 16 * kb, dt * 32, lane), S[i]);
      }
    }
    if constexpr (PHI) {
      if (more && wave >= 4) phi_partial();
    }
    __syncthreads();
    // ---- publish S^T; next chunk into LDS (PHI: its fq from the statistics
    // of phase 2); z update --------------------------------------------------
    publish();
    if (more) {
      if constexpr (PHI)
        phi_write(t0 + C);
      else
        store_chunk512<FP>(rq, fq_l, PF);
      store_chunk512<FP>(rk, fk_l, PF);
      store_chunk512<DP>(rv, v_l, PD);
      if (wave == 0) gate_scan(rg, lane, lgs, qs, ks, rdec, gate, t0 + C + lane < L);
    }
    if (tid < FP) zs[tid] = zs[tid] * r_n + sum_parts<FP>(zp, tid);
    __syncthreads();
  }

  // the state after the whole sequence, [F][D] fp32 then z [F], for decoding
  if (final_state && seg + M == G) {
    float* fs = final_state + (size_t)bh * ((size_t)F * D + F);
#pragma unroll
    for (int i = 0; i < S_OWN; ++i) {
      const int t = wave + 8 * i, ft = t % NFT, dt = t / NFT;
      if (t < NFT * NDT) {
        const int d = dt * 32 + col;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int f = ft * 32 + acc_row(r, h);
          if (f < F && d < D) fs[(size_t)f * D + d] = S[i][r];
        }
      }
    }
    for (int f = tid; f < F; f += WIDE_THREADS) fs[(size_t)F * D + f] = zs[f];
  }
}

// ----------------------------------------------------------------------------
// decode step: one token per (b, h) on the recurrent form
//   S <- gamma S + fk v^T,  z <- gamma z + fk,  y = fq S / max(fq . z, FLT_MIN)
// (tests/test_lizard.py:41-52 of the reference), state [F][D] fp32 then z [F]
// per (b, h), updated in place; fk and v of query head bh are row bh / KG
// (its kv head).  Thread (g, d) of the 256 walks features
// f = g, g + NG, ... of column d (NG = 256 / DP groups); the fq . S_new partial
// sums of the groups meet in LDS.
// ----------------------------------------------------------------------------
template <int DP>
__global__ __launch_bounds__(256) void gla_decode_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, float* __restrict__ state, bf16* __restrict__ y, int H,
    int F, int D, int gate, int KG) {
  constexpr int NG = 256 / DP;
  __shared__ float fq_s[256], fk_s[256], part[256], red[4];
  const int bh = blockIdx.x, tid = threadIdx.x;
  const int g = tid / DP, d = tid % DP;
  const float gam = fexp(gate_log(log_gamma[(gate & GATE_PER_HEAD) ? bh : bh / H], gate));
  const bf16* fqb = fq + (size_t)bh * F;
  const bf16* fkb = fk + (size_t)(bh / KG) * F;
  float* Sb = state + (size_t)bh * ((size_t)F * D + F);
  float* zb = Sb + (size_t)F * D;
  for (int f = tid; f < F; f += 256) {
    fq_s[f] = to_f32(fqb[f]);
    fk_s[f] = to_f32(fkb[f]);
  }
  __syncthreads();
  // z and fq . z
  float qz = 0.f;
  for (int f = tid; f < F; f += 256) {
    const float zn = gam * zb[f] + fk_s[f];
    zb[f] = zn;
    qz += fq_s[f] * zn;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) qz += __shfl_xor(qz, off);
  if ((tid & 63) == 0) red[tid >> 6] = qz;
  // S and fq . S
  float num = 0.f;
  if (d < D) {
    const float vd = to_f32(v[(size_t)(bh / KG) * D + d]);
    for (int f = g; f < F; f += NG) {
      const float sn = gam * Sb[(size_t)f * D + d] + fk_s[f] * vd;
      Sb[(size_t)f * D + d] = sn;
      num += fq_s[f] * sn;
    }
  }
  part[tid] = num;
  __syncthreads();
  if (g == 0 && d < D) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NG; ++j) s += part[j * DP + d];
    const float den = (red[0] + red[1]) + (red[2] + red[3]);
    y[(size_t)bh * D + d] = to_bf16(s / fmaxf(den, TINY));
  }
}

// Vector form of the decode step, for F % 4 == 0 and D a power of two in
// [4, 128] (so S rows and each (b, h) state are 16-byte aligned and the
// quads of a row divide a wave).  512 threads per (b, h): thread t owns
// column quad q = t % (D/4) of rows f = t / (D/4) + i * RG (RG = 512 / (D/4)),
// IPT rows in all.  Every state load of a thread is issued before any use,
// through a range-checked buffer (rows past F read zeros, their stores drop).
// fq . S_new sums over a wave's lanes of the same quad by xor shuffles, then
// over the 8 waves in LDS.
template <int IPT>
__global__ __launch_bounds__(512) void gla_decode_vec_kernel(
    const bf16* __restrict__ fq, const bf16* __restrict__ fk, const bf16* __restrict__ v,
    const float* __restrict__ log_gamma, float* __restrict__ state, bf16* __restrict__ y, int H,
    int F, int D, int gate, int KG) {
  __shared__ float fq_s[256], fk_s[256], red[8];
  __shared__ f32x4 part[8 * 32];
  const int bh = blockIdx.x, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int NQ = D >> 2, RG = 512 / NQ;
  const int q = tid % NQ, r0 = tid / NQ;
  float* Sb = state + (size_t)bh * ((size_t)F * D + F);
  float* zb = Sb + (size_t)F * D;
  const rsrc_t sr = make_rsrc(Sb, (size_t)F * D * 4);
  auto soff = [&](int i) {
    const int f = r0 + i * RG;
    return f < F ? (uint32_t)(f * D + 4 * q) * 4u : OOB;
  };
  f32x4 s[IPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i) s[i] = __builtin_bit_cast(f32x4, bload16(sr, soff(i)));
  const float gam = fexp(gate_log(log_gamma[(gate & GATE_PER_HEAD) ? bh : bh / H], gate));
  for (int f = tid; f < F; f += 512) {
    fq_s[f] = to_f32(fq[(size_t)bh * F + f]);
    fk_s[f] = to_f32(fk[(size_t)(bh / KG) * F + f]);
  }
  const bf16x4 v4 = *reinterpret_cast<const bf16x4*>(v + (size_t)(bh / KG) * D + 4 * q);
  __syncthreads();
  float qz = 0.f;
  for (int f = tid; f < F; f += 512) {
    const float zn = gam * zb[f] + fk_s[f];
    zb[f] = zn;
    qz += fq_s[f] * zn;
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) qz += __shfl_xor(qz, off);
  if (lane == 0) red[wave] = qz;
  f32x4 num = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int f = min(r0 + i * RG, F - 1);   // rows past F: zeros in, store dropped
    const float a = fk_s[f], b = fq_s[f];
    f32x4 sn;
#pragma unroll
    for (int e = 0; e < 4; ++e) sn[e] = gam * s[i][e] + a * to_f32(v4[e]);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sn), sr, soff(i), 0, 0);
    if (r0 + i * RG < F) {
#pragma unroll
      for (int e = 0; e < 4; ++e) num[e] += b * sn[e];
    }
  }
  for (int off = NQ; off < 64; off <<= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) num[e] += __shfl_xor(num[e], off);
  if (lane < NQ) part[wave * 32 + lane] = num;
  __syncthreads();
  if (tid < NQ) {
    f32x4 t = part[tid];
#pragma unroll
    for (int w = 1; w < 8; ++w)
#pragma unroll
      for (int e = 0; e < 4; ++e) t[e] += part[w * 32 + tid][e];
    float den = red[0];
#pragma unroll
    for (int w = 1; w < 8; ++w) den += red[w];
    const float inv = 1.f / fmaxf(den, TINY);
    const bf16x4 o = {to_bf16(t[0] * inv), to_bf16(t[1] * inv), to_bf16(t[2] * inv),
                      to_bf16(t[3] * inv)};
    *reinterpret_cast<bf16x4*>(y + (size_t)bh * D + 4 * tid) = o;
  }
}

hipError_t launch_gla_decode(const void* fq, const void* fk, const void* v, const float* lg,
                             float* state, void* y, int B, int H, int F, int D,
                             int gate, int KG, hipStream_t st) {
  if (F % 4 == 0 && D >= 4 && D <= 128 && (D & (D - 1)) == 0) {
    const int rg = 512 / (D / 4), need = (F + rg - 1) / rg;   // rows per thread
#define LZ_GLA_DECV(IPTV)                                                                     \
    if (need <= IPTV) {                                                                       \
      hipLaunchKernelGGL(gla_decode_vec_kernel<IPTV>, dim3(B * H), dim3(512), 0, st,          \
                         (const bf16*)fq, (const bf16*)fk, (const bf16*)v, lg, state,         \
                         (bf16*)y, H, F, D, gate, KG);                               \
      return hipGetLastError();                                                               \
    }
    LZ_GLA_DECV(1) LZ_GLA_DECV(2) LZ_GLA_DECV(4) LZ_GLA_DECV(8)
#undef LZ_GLA_DECV
  }
  const int dp = D <= 32 ? 32 : (D <= 64 ? 64 : (D <= 128 ? 128 : 256));
#define LZ_GLA_DEC(DPV)                                                                       \
  if (dp == DPV) {                                                                          \
    hipLaunchKernelGGL(gla_decode_kernel<DPV>, dim3(B * H), dim3(256), 0, st,                 \
                       (const bf16*)fq, (const bf16*)fk, (const bf16*)v, lg, state, (bf16*)y, \
                       H, F, D, gate, KG);                                           \
    return hipGetLastError();                                                               \
  }
  LZ_GLA_DEC(32) LZ_GLA_DEC(64) LZ_GLA_DEC(128) LZ_GLA_DEC(256)
#undef LZ_GLA_DEC
  return hipErrorInvalidValue;
}

// ----------------------------------------------------------------------------
// segment pass: state left by each segment g < G-1 starting from zero
// ----------------------------------------------------------------------------
// Its LDS: only the fk and v tiles of a chunk and the gate and z scratch
// (no fq, no score fragments), so two workgroups fit a CU at every F.
template <int FP, int DP>
struct GlaState {
  static constexpr int C = GLA_C;
  static constexpr int PF = lds_pitch(FP), PD = lds_pitch(DP);
  static constexpr int NFT = FP / 32, NDT = DP / 32;
  static constexpr int NLF = C * FP / 8 / 256;        // 16-byte loads per thread, fk
  static constexpr int NLD = C * DP / 8 / 256;        // 16-byte loads per thread, v
  static constexpr int OFF_FK = 0;
  static constexpr int OFF_V = OFF_FK + C * PF * 2;
  // gate arrays, decays and K~ column sums, one set per chunk parity
  static constexpr int OFF_LG = OFF_V + C * PD * 2;       // [2][64] chunk-local lg
  static constexpr int OFF_QS = OFF_LG + 2 * 64 * 4;      // [2][64] e^{lg} (written by gate_scan)
  static constexpr int OFF_KS = OFF_QS + 2 * 64 * 4;      // [2][64] e^{lg_end - lg}
  static constexpr int OFF_Z = OFF_KS + 2 * 64 * 4;       // [FP] z
  static constexpr int OFF_ZP = OFF_Z + FP * 4;           // [2][2048] partial sums of K~
  static constexpr int OFF_R = OFF_ZP + 2 * 2048 * 4;     // [2][4] e^{lg_end}, lg_end
  static constexpr int BYTES = OFF_R + 32;
  static constexpr int SEG = SegRec<FP, DP>::SIZE;
  static_assert(BYTES <= 80 * 1024, "LDS budget: two workgroups per CU");
};

// Columns [0, ncols) of chunk rows t0 .. t0 + 63 of a row-major bf16 matrix
// whose rows are `stride` elements apart, behind a buffer of `bytes` bytes from
// `base` (rows past it read zeros); the item layout of load_chunk.
template <int KP, int N>
__device__ __forceinline__ void load_chunk_strided(uint4 (&reg)[N], const bf16* __restrict__ base,
                                                   size_t bytes, int t0, int stride, int ncols,
                                                   bool vec) {
  constexpr int K8 = KP / 8;
  const rsrc_t r = make_rsrc(base, bytes);
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int idx = threadIdx.x + 256 * i;
    const int row = t0 + idx / K8, c = (idx % K8) * 8;
    if (vec) {
      reg[i] = bload16(r, c < ncols ? (uint32_t)(row * stride + c) * 2u : OOB);
    } else {
      bf16x8 x;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t off = c + e < ncols ? (uint32_t)(row * stride + c + e) * 2u : OOB;
        x[e] = __builtin_bit_cast(bf16, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
      }
      reg[i] = __builtin_bit_cast(uint4, x);
    }
  }
}

// FR: the record's padded feature count.  FP < FR splits the state's feature
// rows over FR / FP workgroups per segment: row f of S and z[f] depend only on
// column f of fk, so each takes its slice of fk's columns (and all of v) and
// writes its rows of the record.  Used when the segments alone leave most of
// the GPU idle (few kv heads with a shared gate).
template <int FP, int DP, bool VEC, int FR, bool REV = false>
__global__ __launch_bounds__(256, 2) void gla_fwd_state_kernel(
    const bf16* __restrict__ fk, const bf16* __restrict__ v, const float* __restrict__ log_gamma,
    float* __restrict__ seg_state, float* __restrict__ seg_logdecay, int H, int L, int F, int D,
    int gate, int G, int cps, int KG) {
  using Cfg = GlaState<FP, DP>;
  constexpr int C = Cfg::C, PF = Cfg::PF, PD = Cfg::PD;
  constexpr int NFT = Cfg::NFT, NDT = Cfg::NDT;
  constexpr int NTILE = NFT * NDT;
  constexpr int TPW = (NTILE + 3) / 4;   // state tiles per wave
  extern __shared__ __align__(16) char smem[];
  bf16* fk_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_FK);
  bf16* v_l = reinterpret_cast<bf16*>(smem + Cfg::OFF_V);
  float* lgs = reinterpret_cast<float*>(smem + Cfg::OFF_LG);
  float* qs = reinterpret_cast<float*>(smem + Cfg::OFF_QS);
  float* ks = reinterpret_cast<float*>(smem + Cfg::OFF_KS);
  float* zs = reinterpret_cast<float*>(smem + Cfg::OFF_Z);
  float* zp = reinterpret_cast<float*>(smem + Cfg::OFF_ZP);
  float* rdec = reinterpret_cast<float*>(smem + Cfg::OFF_R);

  constexpr int NFS = FR / FP;
  static_assert(FR % FP == 0, "feature slices divide the record");
  const int fs = NFS > 1 ? (int)(blockIdx.x % NFS) : 0, f0 = fs * FP;
  const int blk = NFS > 1 ? (int)(blockIdx.x / NFS) : (int)blockIdx.x;
  const int bh = blk / (G - 1), seg = blk % (G - 1);
  const int n0 = seg * cps, n1 = n0 + cps;   // segments before the last are full
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int col = lane & 31, h = lane >> 5;
  const bool vecF = VEC || (F & 7) == 0, vecD = VEC || (D & 7) == 0;
  // this workgroup's columns f0 .. f0 + FP - 1 of fk (rows F apart)
  const bf16* fkb = fk + (size_t)(bh / KG) * L * F + f0;
  const int fcols = F - f0;   // valid columns from f0 (<= 0: none, the slice is zero)
  const size_t fk_bytes = fcols > 0 ? ((size_t)L * F - f0) * 2 : 0;
  const bf16* vb = v + (size_t)(bh / KG) * L * D;
  const float* lgb = log_gamma + (size_t)((gate & GATE_PER_HEAD) ? bh : bh / H) * L;
  auto load_fk = [&](uint4 (&reg)[Cfg::NLF], int t) {
    if constexpr (NFS == 1)
      load_chunk<FP>(reg, fkb, t, L, F, vecF);
    else
      load_chunk_strided<FP>(reg, fkb, fk_bytes, t, F, fcols, vecF);
  };

  f32x16 S[TPW];
#pragma unroll
  for (int i = 0; i < TPW; ++i) S[i] = zero16();
  for (int f = tid; f < FP; f += 256) zs[f] = 0.f;
  float lam = 0.f;   // total log decay of the segment (wave 0)

  // fk is staged as K~ = bf16(fk ks): each thread scales its prefetched
  // 16-byte items (the item layout of scale_rows) by the staged chunk's ks
  // and writes their column sums, so the state update reads ready operands.
  // That needs the chunk's gate scan before it is staged: wave 0 scans the
  // next chunk's gates while the current one updates the state, into the
  // buffers of the other chunk parity.
  using R = RowItems<FP>;
  static_assert(Cfg::NLF == R::N, "chunk items follow the scale_rows layout");
  const int cg = tid % R::K8, r0 = tid / R::K8;
  auto stage_scaled = [&](const uint4 (&reg)[Cfg::NLF], const float* kss, float* part) {
    float sum[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) sum[e] = 0.f;
#pragma unroll
    for (int i = 0; i < R::N; ++i) {
      const int t = r0 + R::RSTRIDE * i;
      const bf16x8 x = __builtin_bit_cast(bf16x8, reg[i]);
      const float sc = kss[t];
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o[e] = to_bf16(to_f32(x[e]) * sc);
        sum[e] += to_f32(o[e]);
      }
      *reinterpret_cast<bf16x8*>(fk_l + t * PF + 8 * cg) = o;
    }
    if constexpr (NFS == 1) {
      float* dst = part + r0 * FP + 8 * cg;
      *reinterpret_cast<f32x4*>(dst) = f32x4{sum[0], sum[1], sum[2], sum[3]};
      *reinterpret_cast<f32x4*>(dst + 4) = f32x4{sum[4], sum[5], sum[6], sum[7]};
    }
  };
  // A feature slice (NFS > 1) sums the staged chunk's K~ columns for z in the
  // order the FR-wide layout does (RowItems<FR>: partial p over rows p, p + RS,
  // p + 2 RS, ..., then the partials in turn), so that a record's bits do not
  // depend on how its rows were split.
  using RR = RowItems<FR>;
  static_assert(RR::PARTS * FP <= 2048, "a slice's partial sums fit one parity of zp");
  auto slice_parts = [&](float* part) {
    for (int task = tid; task < RR::PARTS * FP; task += 256) {
      const int p = task / FP, c = task % FP;
      float q = 0.f;
#pragma unroll
      for (int i = 0; i < RR::N; ++i) q += to_f32(fk_l[(p + RR::RSTRIDE * i) * PF + c]);
      part[p * FP + c] = q;
    }
  };

  // REV walks the segment from its last chunk to its first: the record is
  // S = sum_n dec_n K~_n^T V_n with dec_n the decay from the end of chunk n to
  // the end of the segment (the product of the later chunks' decays), so each
  // chunk's product is formed from zero and added scaled by dec_n.  The walk
  // that follows reads each segment from its first chunk, which this pass then
  // read last: when the segments' rows are more than the memory-side cache
  // holds, those rows are the ones still in it as the walk starts (read in the
  // walk's order, the walk's first rows are the first ones evicted).
  uint4 rk[Cfg::NLF], rv[Cfg::NLD];
  const int nf = REV ? n1 - 1 : n0;   // the first chunk this pass reads
  float rg = gate_at(lgb, nf * C + lane, L);   // the gate first: waited for alone
  load_fk(rk, nf * C);
  load_chunk<DP>(rv, vb, nf * C, L, D, vecD);
  {
    const int pb = nf & 1;
    if (wave == 0)
      gate_scan(rg, lane, lgs + 64 * pb, qs + 64 * pb, ks + 64 * pb, rdec + 4 * pb, gate,
                nf * C + lane < L);
    __syncthreads();
    stage_scaled(rk, ks + 64 * pb, zp + 2048 * pb);
    store_chunk<DP>(rv, v_l, PD);
    __syncthreads();
  }

  float dec = 1.f;   // REV: decay from the end of chunk n to the end of the segment
  for (int n = nf; REV ? n >= n0 : n < n1; n += REV ? -1 : 1) {
    const int t0 = n * C;
    const bool more = REV ? n > n0 : n + 1 < n1;
    const int pc = n & 1, pn = pc ^ 1;   // this chunk's parity, the next one's
    // unconditional loads (past the segment they read rows past L: zeros, no
    // traffic), so the scan below waits for the gate alone
    const int tn = more ? (REV ? t0 - C : t0 + C) : L;
    rg = gate_at(lgb, tn + lane, L);
    load_fk(rk, tn);
    load_chunk<DP>(rv, vb, tn, L, D, vecD);
    __builtin_amdgcn_s_setprio(0);
    const float r_n = rdec[4 * pc];
    if (wave == 0) lam += rdec[4 * pc + 1];
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int ti = wave + 4 * i;
      if (ti < NTILE) {
        const int ft = ti / NDT, dt = ti % NDT;
        if constexpr (REV) {
          f32x16 T = zero16();
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
            T = mfma(tr_operand(fk_l, PF, 16 * kb, ft * 32, lane),
                     tr_operand(v_l, PD, 16 * kb, dt * 32, lane), T);
#pragma unroll
          for (int r = 0; r < 16; ++r) S[i][r] = __builtin_fmaf(dec, T[r], S[i][r]);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) S[i][r] *= r_n;
#pragma unroll
          for (int kb = 0; kb < 4; ++kb)
            S[i] = mfma(tr_operand(fk_l, PF, 16 * kb, ft * 32, lane),
                        tr_operand(v_l, PD, 16 * kb, dt * 32, lane), S[i]);
        }
      }
    }
    if constexpr (NFS > 1) slice_parts(zp + 2048 * pc);
    if (more && wave == 0)
      gate_scan(rg, lane, lgs + 64 * pn, qs + 64 * pn, ks + 64 * pn, rdec + 4 * pn, gate,
                tn + lane < L);
    __syncthreads();
    // staging and the next loads at raised wave priority, as in the walk
    __builtin_amdgcn_s_setprio(1);
    if constexpr (NFS == 1) {
      if (tid < FP) {
        if constexpr (REV)
          zs[tid] = __builtin_fmaf(dec, sum_parts<FP>(zp + 2048 * pc, tid), zs[tid]);
        else
          zs[tid] = zs[tid] * r_n + sum_parts<FP>(zp + 2048 * pc, tid);
      }
    } else if (tid < FP) {
      float zc = 0.f;
      for (int p = 0; p < RR::PARTS; ++p) zc += zp[2048 * pc + p * FP + tid];
      zs[tid] = REV ? __builtin_fmaf(dec, zc, zs[tid]) : zs[tid] * r_n + zc;
    }
    if constexpr (REV) dec *= r_n;
    if (more) {
      stage_scaled(rk, ks + 64 * pn, zp + 2048 * pn);
      store_chunk<DP>(rv, v_l, PD);
    }
    __syncthreads();
  }
  float* out = seg_state + ((size_t)bh * G + seg) * SegRec<FR, DP>::SIZE;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int ti = wave + 4 * i;
    if (ti < NTILE) {
      const int ft = ti / NDT, dt = ti % NDT;
#pragma unroll
      for (int r = 0; r < 16; ++r)
        out[(f0 + ft * 32 + acc_row(r, h)) * DP + dt * 32 + col] = S[i][r];
    }
  }
  for (int f = tid; f < FP; f += 256) out[FR * DP + f0 + f] = zs[f];
  if (tid == 0 && fs == 0) seg_logdecay[(size_t)bh * G + seg] = lam;
}

// ----------------------------------------------------------------------------
// exclusive scan over segments, in place.  Forward (reverse == 0): record g
// holds the state segment g leaves from zero (g < G-1) and becomes the state
// entering segment g.  Reverse: record g holds the gradient state segment g
// leaves (walking backwards) from zero (g > 0) and becomes the gradient state
// entering segment g from the right.  seg_logdecay[g] is segment g's total
// log decay.
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gla_segment_scan_kernel(float* __restrict__ seg_state,
                                                               const float* __restrict__ seg_logdecay,
                                                               int G, int rec, int reverse) {
  const int bh = blockIdx.y;
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= rec) return;
  float* base = seg_state + (size_t)bh * G * rec + e;
  const float* lam = seg_logdecay + (size_t)bh * G;
  float carry = 0.f;
  // records are read in batches of 8 independent loads, then combined in order
  for (int b0 = 0; b0 < G - 1; b0 += 8) {
    float d[8], w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int g = reverse ? G - 1 - (b0 + k) : b0 + k;
      const bool ok = b0 + k < G - 1;
      d[k] = ok ? base[(size_t)g * rec] : 0.f;
      w[k] = ok ? fexp(lam[g]) : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (b0 + k < G - 1) {
        const int g = reverse ? G - 1 - (b0 + k) : b0 + k;
        base[(size_t)g * rec] = carry;
        carry = __builtin_fmaf(w[k], carry, d[k]);   // as fold_records
      }
    }
  }
  base[(size_t)(reverse ? 0 : G - 1) * rec] = carry;
}

// ----------------------------------------------------------------------------
// host side
// ----------------------------------------------------------------------------
int gla_padded_dim(int n) {
  if (n <= 32) return 32;
  if (n <= 64) return 64;
  if (n <= 128) return 128;
  if (n <= 256) return 256;
  return -1;
}

bool gla_dims_supported(int F, int D) {
  const int fp = gla_padded_dim(F), dp = gla_padded_dim(D);
  if (fp < 0 || dp < 0) return false;
  return dp <= 128 && (fp <= 128 || dp <= 64);
}

// Segments per (b, h) so that B*H*G workgroups fill the GPU: two forward
// workgroups per CU up to F = 128, one beyond (the LDS of a 256-wide chunk).
void gla_segments(int BH, int L, int F, int* G, int* cps) {
  const int NT = (L + GLA_C - 1) / GLA_C;
  const bool wide = gla_padded_dim(F) > 128;   // walks run one workgroup per CU
  const int target = wide ? gla_target_wg() / 2 : gla_target_wg();
  int g = (target + BH - 1) / BH;
  g = g < 1 ? 1 : (g > NT ? NT : g);
  // Wide walks: segments half as long as one walk, each walk taking two
  // (gla_walk_segments).  The segment state passes, which fit two workgroups
  // per CU, then run twice the workgroups at half the length.
  if (wide && g > 1) g = 2 * g > NT ? NT : 2 * g;
  const int c = (NT + g - 1) / g;
  *cps = c;
  *G = (NT + c - 1) / c;
}

// Segments one walk workgroup takes in a row: two when each (b, h) has an
// even number of segments and half as many workgroups still fill the GPU at
// one per CU (wide walks; the segment split doubled for them).
int gla_walk_segments(int BH, int G, int F) {
  return gla_padded_dim(F) > 128 && G % 2 == 0 && BH * G / 2 >= gla_target_wg() / 2 ? 2 : 1;
}

// workspace floats of one segment-state set: records + log decays
size_t gla_segment_floats(int BH, int G, int F, int D) {
  if (G <= 1) return 0;
  const size_t rec = (size_t)gla_padded_dim(F) * gla_padded_dim(D) + gla_padded_dim(F);
  return (size_t)BH * G * rec + (size_t)BH * G;
}

size_t gla_fwd_workspace(int B, int H, int L, int F, int D) {
  int G, cps;
  gla_segments(B * H, L, F, &G, &cps);
  return gla_segment_floats(B * H, G, F, D) * sizeof(float);
}

hipError_t launch_gla_segment_scan(float* seg_state, const float* seg_logdecay, int BH, int G,
                                   int rec, bool reverse, hipStream_t st) {
  hipLaunchKernelGGL(gla_segment_scan_kernel, dim3((rec + 255) / 256, BH), dim3(256), 0, st,
                     seg_state, seg_logdecay, G, rec, reverse ? 1 : 0);
  return hipGetLastError();
}

// The state pass reads its segments' chunks from the last to the first (REV)
// when those rows are more than half of the memory-side cache (256 MB on
// MI355X), so that the walk starts on rows still cached; below that both
// orders leave the rows cached and the forward loop is the cheaper one.
constexpr size_t GLA_STATE_REV_BYTES = size_t(128) << 20;

// the state pass with the record's FR feature rows in slices of FS per
// workgroup; rev: the reverse chunk order (unsliced passes only: a sliced pass
// has few segments, whose rows the cache holds)
template <int FS, int FR, int DP, bool VEC>
static hipError_t launch_state_slices(const void* fk, const void* v, const float* lg,
                                      float* seg_state, float* seg_logdecay, int BH, int H, int L,
                                      int F, int D, int gate, int G, int cps, int KG, bool rev,
                                      hipStream_t st) {
  using Cfg = GlaState<FS, DP>;
  auto launch = [&](auto tag) {
    constexpr auto kern = decltype(tag)::value;
    if (hipError_t e = ensure_lds<kern>(Cfg::BYTES); e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(BH * (G - 1) * (FR / FS)), dim3(256), Cfg::BYTES, st,
                       (const bf16*)fk, (const bf16*)v, lg, seg_state, seg_logdecay, H, L, F, D,
                       gate, G, cps, KG);
    return hipGetLastError();
  };
  if constexpr (FS == FR)
    if (rev) return launch(KernTag<gla_fwd_state_kernel<FS, DP, VEC, FR, true>>{});
  return launch(KernTag<gla_fwd_state_kernel<FS, DP, VEC, FR>>{});
}

// Feature slices per segment: doubled while the state pass would still fill
// at most half of the GPU's two workgroups per CU, down to 64 features.
static int gla_state_slices(int workgroups, int FP) {
  int n = 1;
  while (n < FP / 64 && workgroups * n * 2 <= gla_target_wg()) n *= 2;
  return n;
}

template <int FP, int DP, bool VEC>
static hipError_t launch_gla_fwd_states_t(const void* fk, const void* v, const float* lg,
                                          float* seg_state, float* seg_logdecay, int BH, int H,
                                          int L, int F, int D, int gate, int G, int cps,
                                          int KG, bool fold, hipStream_t st) {
  if (!(gate & GATE_PER_HEAD) && KG > 1) {   // one record per kv head (seg_owner)
    BH /= KG;
    H /= KG;
    KG = 1;
  }
  const int nfs = gla_state_slices(BH * (G - 1), FP);
  // the fk and v rows the pass reads (all segments but the last)
  const size_t rows_bytes = (size_t)BH * (G - 1) * cps * GLA_C * (size_t)(F + D) * 2;
  const bool rev = rows_bytes > GLA_STATE_REV_BYTES;
  hipError_t e;
  if constexpr (FP == 256) {
    if (nfs == 4)
      e = launch_state_slices<64, FP, DP, VEC>(fk, v, lg, seg_state, seg_logdecay, BH, H, L, F,
                                               D, gate, G, cps, KG, rev, st);
    else if (nfs == 2)
      e = launch_state_slices<128, FP, DP, VEC>(fk, v, lg, seg_state, seg_logdecay, BH, H, L, F,
                                                D, gate, G, cps, KG, rev, st);
    else
      e = launch_state_slices<FP, FP, DP, VEC>(fk, v, lg, seg_state, seg_logdecay, BH, H, L, F,
                                               D, gate, G, cps, KG, rev, st);
  } else if constexpr (FP == 128) {
    if (nfs == 2)
      e = launch_state_slices<64, FP, DP, VEC>(fk, v, lg, seg_state, seg_logdecay, BH, H, L, F,
                                               D, gate, G, cps, KG, rev, st);
    else
      e = launch_state_slices<FP, FP, DP, VEC>(fk, v, lg, seg_state, seg_logdecay, BH, H, L, F,
                                               D, gate, G, cps, KG, rev, st);
  } else {
    e = launch_state_slices<FP, FP, DP, VEC>(fk, v, lg, seg_state, seg_logdecay, BH, H, L, F, D,
                                             gate, G, cps, KG, rev, st);
  }
  if (e != hipSuccess) return e;
  if (fold) return hipSuccess;   // the walks fold the records
  return launch_gla_segment_scan(seg_state, seg_logdecay, BH, G, SegRec<FP, DP>::SIZE, false,
                                 st);
}

hipError_t launch_gla_fwd_states(const void* fk, const void* v, const float* lg, float* seg_state,
                                 float* seg_logdecay, int BH, int H, int L, int F, int D,
                                 int gate, int G, int cps, int KG, bool fold, hipStream_t st) {
  const int fp = gla_padded_dim(F), dp = gla_padded_dim(D);
  const bool vec = F % 8 == 0 && D % 8 == 0;
#define LZ_GLA_ST(FPV, DPV)                                                                   \
  if (fp == FPV && dp == DPV)                                                                 \
    return vec ? launch_gla_fwd_states_t<FPV, DPV, true>(fk, v, lg, seg_state, seg_logdecay,  \
                                                         BH, H, L, F, D, gate, G,    \
                                                         cps, KG, fold, st)                   \
               : launch_gla_fwd_states_t<FPV, DPV, false>(fk, v, lg, seg_state, seg_logdecay, \
                                                          BH, H, L, F, D, gate, G,   \
                                                          cps, KG, fold, st);
  LZ_GLA_ST(32, 32) LZ_GLA_ST(32, 64) LZ_GLA_ST(32, 128)
  LZ_GLA_ST(64, 32) LZ_GLA_ST(64, 64) LZ_GLA_ST(64, 128)
  LZ_GLA_ST(128, 32) LZ_GLA_ST(128, 64) LZ_GLA_ST(128, 128)
  LZ_GLA_ST(256, 32) LZ_GLA_ST(256, 64)
#undef LZ_GLA_ST
  return hipErrorInvalidValue;
}

template <int FP, int DP, bool VEC, bool RAW>
static hipError_t launch_gla_fwd_t(const void* fq, const void* fk, const void* v,
                                   const float* lg, void* y, int B, int H, int L, int F, int D,
                                   int gate, int KG, float* ws, float* final_state,
                                   float* raw_den, hipStream_t st) {
  using Cfg = GlaFwd<FP, DP>;
  const int BH = B * H;
  int G, cps;
  gla_segments(BH, L, F, &G, &cps);
  constexpr bool CAN_FOLD = gla_can_fold<FP, DP, VEC>() && !RAW;
  const bool fold = CAN_FOLD && gla_fold_segments(G);
  float* seg_state = ws;
  float* seg_lam = ws + (size_t)BH * G * Cfg::SEG;
  if (G > 1) {
    hipError_t e = launch_gla_fwd_states_t<FP, DP, VEC>(fk, v, lg, seg_state, seg_lam, BH, H, L,
                                                        F, D, gate, G, cps, KG, fold, st);
    if (e != hipSuccess) return e;
  }
  const int M = gla_walk_segments(BH, G, F);
  const WalkGrid wg = walk_grid(BH * G / M, KG);
  if constexpr (FP == 256) {   // eight waves per workgroup
    using W = GlaFwdWide<DP>;
    auto launch = [&](auto tag) {
      constexpr auto kern = decltype(tag)::value;
      hipError_t e = ensure_lds<kern>(W::BYTES);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(kern, dim3(wg.grid), dim3(WIDE_THREADS), W::BYTES, st,
                         (const bf16*)fq, (const bf16*)fk, (const bf16*)v, lg, (bf16*)y,
                         (const float*)seg_state, final_state, H, L, F, D, gate, G, cps, M, KG,
                         RAW ? (float*)y : nullptr, raw_den, wg.per, wg.nx, wg.nblk,
                         (const bf16*)nullptr, (const bf16*)nullptr, (const float*)seg_lam);
      return hipGetLastError();
    };
    if constexpr (CAN_FOLD)
      if (fold) return launch(KernTag<gla_fwd_wide_kernel<DP, VEC, RAW, false, true>>{});
    return launch(KernTag<gla_fwd_wide_kernel<DP, VEC, RAW, false>>{});
  } else {
    auto launch = [&](auto tag) {
      constexpr auto kern = decltype(tag)::value;
      hipError_t e = ensure_lds<kern>(Cfg::BYTES);
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL(kern, dim3(wg.grid), dim3(256), Cfg::BYTES, st, (const bf16*)fq,
                         (const bf16*)fk, (const bf16*)v, lg, (bf16*)y, (const float*)seg_state,
                         final_state, H, L, F, D, gate, G, cps, M, KG,
                         RAW ? (float*)y : nullptr, raw_den, wg.per, wg.nx, wg.nblk,
                         (const float*)seg_lam);
      return hipGetLastError();
    };
    if constexpr (CAN_FOLD)
      if (fold) return launch(KernTag<gla_fwd_kernel<FP, DP, VEC, RAW, true>>{});
    // the caller reads fq, fk, v no more (GATE_NO_REUSE: no backward
    // follows), and with one segment and no kv head shared by query heads
    // this walk reads each row once: its chunk loads go nontemporal
    // (headline forward 216.9 -> 208.8 us).  Where a state pass or other
    // heads' walks read the rows again, as at config 2, such loads were 15 %
    // slower, and before a backward the fwd+bwd was 0.5 % slower.
    if constexpr (VEC && !RAW)
      if ((gate & GATE_NO_REUSE) && G == 1 && KG == 1)
        return launch(KernTag<gla_fwd_kernel<FP, DP, VEC, RAW, false, true>>{});
    return launch(KernTag<gla_fwd_kernel<FP, DP, VEC, RAW>>{});
  }
}

// The LDS limit (hipFuncSetAttribute) of every kernel launch_gla_fwd and
// launch_gla_fwd_states can launch at the walks' own sizes, set on the
// current device; afterwards those launches make no other runtime call.
template <int FP, int DP, bool VEC>
static hipError_t prepare_fwd_t() {
  hipError_t e;
  if constexpr (FP == 256)
    e = ensure_lds<gla_fwd_wide_kernel<DP, VEC, false, false>>(GlaFwdWide<DP>::BYTES);
  else
    e = ensure_lds<gla_fwd_kernel<FP, DP, VEC, false>>(GlaFwd<FP, DP>::BYTES);
  if (e != hipSuccess) return e;
  if constexpr (gla_can_fold<FP, DP, VEC>()) {   // the folding walks
    if constexpr (FP == 256)
      e = ensure_lds<gla_fwd_wide_kernel<DP, VEC, false, false, true>>(GlaFwdWide<DP>::BYTES);
    else
      e = ensure_lds<gla_fwd_kernel<FP, DP, VEC, false, true>>(GlaFwd<FP, DP>::BYTES);
    if (e != hipSuccess) return e;
  }
  if constexpr (FP < 256 && VEC) {   // the walk with nontemporal chunk loads
    e = ensure_lds<gla_fwd_kernel<FP, DP, VEC, false, false, true>>(GlaFwd<FP, DP>::BYTES);
    if (e != hipSuccess) return e;
  }
  if constexpr (FP == 256) {   // the feature-sliced state passes
    if ((e = ensure_lds<gla_fwd_state_kernel<64, DP, VEC, FP>>(GlaState<64, DP>::BYTES)) !=
        hipSuccess)
      return e;
    if ((e = ensure_lds<gla_fwd_state_kernel<128, DP, VEC, FP>>(GlaState<128, DP>::BYTES)) !=
        hipSuccess)
      return e;
  } else if constexpr (FP == 128) {
    if ((e = ensure_lds<gla_fwd_state_kernel<64, DP, VEC, FP>>(GlaState<64, DP>::BYTES)) !=
        hipSuccess)
      return e;
  }
  if ((e = ensure_lds<gla_fwd_state_kernel<FP, DP, VEC, FP, true>>(GlaState<FP, DP>::BYTES)) !=
      hipSuccess)   // the reverse-order pass
    return e;
  return ensure_lds<gla_fwd_state_kernel<FP, DP, VEC, FP>>(GlaState<FP, DP>::BYTES);
}

hipError_t gla_fwd_prepare() {
  hipError_t e;
#define LZ_GLA_PREP(FPV, DPV)                                               \
  if ((e = prepare_fwd_t<FPV, DPV, true>()) != hipSuccess) return e;        \
  if ((e = prepare_fwd_t<FPV, DPV, false>()) != hipSuccess) return e;
  LZ_GLA_PREP(32, 32) LZ_GLA_PREP(32, 64) LZ_GLA_PREP(32, 128)
  LZ_GLA_PREP(64, 32) LZ_GLA_PREP(64, 64) LZ_GLA_PREP(64, 128)
  LZ_GLA_PREP(128, 32) LZ_GLA_PREP(128, 64) LZ_GLA_PREP(128, 128)
  LZ_GLA_PREP(256, 32) LZ_GLA_PREP(256, 64)
#undef LZ_GLA_PREP
  return hipSuccess;
}

// raw_den == nullptr: y is the bf16 output; otherwise (one F tile of a split
// feature dimension) y is the fp32 numerator [BH, L, D] and raw_den the fp32
// denominator [BH, L] of this tile (see gla_fwd_kernel's RAW).
hipError_t launch_gla_fwd(const void* fq, const void* fk, const void* v, const float* lg, void* y,
                          int B, int H, int L, int F, int D, int gate, int KG, float* ws,
                          float* final_state, float* raw_den, hipStream_t st) {
  const int fp = gla_padded_dim(F), dp = gla_padded_dim(D);
  const bool vec = F % 8 == 0 && D % 8 == 0;
#define LZ_GLA_FWD_R(FPV, DPV, V)                                                               \
  (raw_den ? launch_gla_fwd_t<FPV, DPV, V, true>(fq, fk, v, lg, y, B, H, L, F, D,               \
                                                 gate, KG, ws, final_state, raw_den,   \
                                                 st)                                            \
           : launch_gla_fwd_t<FPV, DPV, V, false>(fq, fk, v, lg, y, B, H, L, F, D,              \
                                                  gate, KG, ws, final_state, nullptr,  \
                                                  st))
#define LZ_GLA_FWD(FPV, DPV)                                                                    \
  if (fp == FPV && dp == DPV)                                                                   \
    return vec ? LZ_GLA_FWD_R(FPV, DPV, true) : LZ_GLA_FWD_R(FPV, DPV, false);
  LZ_GLA_FWD(32, 32) LZ_GLA_FWD(32, 64) LZ_GLA_FWD(32, 128)
  LZ_GLA_FWD(64, 32) LZ_GLA_FWD(64, 64) LZ_GLA_FWD(64, 128)
  LZ_GLA_FWD(128, 32) LZ_GLA_FWD(128, 64) LZ_GLA_FWD(128, 128)
  LZ_GLA_FWD(256, 32) LZ_GLA_FWD(256, 64)
#undef LZ_GLA_FWD
#undef LZ_GLA_FWD_R
  return hipErrorInvalidValue;
}

// GLA forward with the feature map of q formed inside the walk (PHI): q rows
// [B, L, H, 64] and W [128][64] bf16 in place of fq; fk [B, H/KG, L, 256],
// v [B, H/KG, L, 64].  Segments, state pass and scan as launch_gla_fwd (the
// state pass reads fk and v only).
hipError_t launch_gla_fwd_phi(const void* q, const void* wq, const void* fk, const void* v,
                              const float* lg, void* y, int B, int H, int L, int gate, int KG,
                              float* ws, float* final_state, hipStream_t st) {
  constexpr int FP = 256, DP = 64;
  const int F = FP, D = DP, BH = B * H;
  int G, cps;
  gla_segments(BH, L, F, &G, &cps);
  float* seg_lam = ws + (size_t)BH * G * GlaFwd<FP, DP>::SEG;
  const bool fold = gla_fold_segments(G);   // the walk with phi has a folding variant
  static_assert(gla_can_fold<FP, DP, true>(), "folding variant of the phi walk");
  if (G > 1) {
    hipError_t e = launch_gla_fwd_states_t<FP, DP, true>(fk, v, lg, ws, seg_lam, BH, H, L, F, D,
                                                         gate, G, cps, KG, fold, st);
    if (e != hipSuccess) return e;
  }
  const int M = gla_walk_segments(BH, G, F);
  const WalkGrid wg = walk_grid(BH * G / M, KG);
  using W = GlaFwdWide<DP>;
  auto launch = [&](auto tag) {
    constexpr auto kern = decltype(tag)::value;
    hipError_t e = ensure_lds<kern>(W::PHI_BYTES);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kern, dim3(wg.grid), dim3(WIDE_THREADS), W::PHI_BYTES, st,
                       (const bf16*)nullptr, (const bf16*)fk, (const bf16*)v, lg, (bf16*)y,
                       (const float*)ws, final_state, H, L, F, D, gate, G, cps, M, KG,
                       (float*)nullptr, (float*)nullptr, wg.per, wg.nx, wg.nblk, (const bf16*)q,
                       (const bf16*)wq, (const float*)seg_lam);
    return hipGetLastError();
  };
  if (fold) return launch(KernTag<gla_fwd_wide_kernel<DP, true, false, true, true>>{});
  return launch(KernTag<gla_fwd_wide_kernel<DP, true, false, true>>{});
}

}  // namespace lz

