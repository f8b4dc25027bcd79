// Pieces shared by the GLA forward and backward kernels: chunk staging,
// the chunk-local gate scan, segment bookkeeping.
#pragma once
#include "common.hpp"

namespace lz {

constexpr int GLA_C = 64;            // chunk length (tokens)
constexpr int GLA_TARGET_WG = 512;   // (b, h, segment) workgroups wanted per launch

int gla_padded_dim(int n);
bool gla_dims_supported(int F, int D);
void gla_segments(int BH, int L, int* G, int* cps);
size_t gla_segment_floats(int BH, int G, int F, int D);

// Rows [t0, t0+64) of a [L x ncols] bf16 matrix into registers, 16 bytes per
// load: thread slot idx = tid + 256 i covers row idx / (KP/8), columns
// 8 * (idx % (KP/8)) .. +8.  Zero outside the matrix.
template <int KP, int N>
__device__ __forceinline__ void load_chunk(uint4 (&reg)[N], const bf16* __restrict__ base, int t0,
                                           int L, int ncols, bool vec) {
  constexpr int K8 = KP / 8;
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const int idx = threadIdx.x + 256 * i;
    reg[i] = gload8(base, t0 + idx / K8, (idx % K8) * 8, L, ncols, vec);
  }
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

// Chunk-local inclusive scan of the gate by one wave (lane = token): lg,
// e^{lg}, e^{lg_end - lg}, and e^{lg_end}, lg_end in r[0], r[1].
__device__ __forceinline__ void gate_scan(float g, int lane, float* lgs, float* qs, float* ks,
                                          float* r) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float o = __shfl_up(g, off);
    if (lane >= off) g += o;
  }
  const float end = __shfl(g, 63);
  lgs[lane] = g;
  qs[lane] = fexp(g);
  ks[lane] = fexp(end - g);
  if (lane == 0) {
    r[0] = fexp(end);
    r[1] = end;
  }
}

__device__ __forceinline__ float gate_at(const float* __restrict__ lgb, int t, int L) {
  return t < L ? lgb[t] : 0.f;
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

// Per-(b, h, segment) state record: S [FP][DP] fp32, then z [FP].
template <int FP, int DP>
struct SegRec {
  static constexpr int SIZE = FP * DP + FP;
};

// Segment pass of the forward recurrence (gla_fwd.hip) and the scan over
// segments; used by the forward and by the backward's forward walk.
hipError_t launch_gla_fwd_states(const void* fk, const void* v, const float* lg, float* seg_state,
                                 float* seg_logdecay, int BH, int H, int L, int F, int D,
                                 int gate_per_head, int G, int cps, hipStream_t st);
hipError_t launch_gla_segment_scan(float* seg_state, const float* seg_logdecay, int BH, int G,
                                   int rec, bool reverse, hipStream_t st);

}  // namespace lz
