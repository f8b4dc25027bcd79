// Shared device helpers for the Lizard attention kernels (gfx950 / CDNA4).
//
// Every contraction is a bf16 MFMA v_mfma_f32_32x32x16_bf16 with fp32
// accumulation.  Operand layout of that instruction (lane l of a 64-wide
// wave, h = l / 32):
//   A (32 x 16):  lane holds row  l % 32, k-slots j = 0..7
//   B (16 x 32):  lane holds col  l % 32, k-slots j = 0..7
//   D (32 x 32):  lane holds col  l % 32, register r holds row acc_row(r, h)
// The hardware pairs k-slot j of A with k-slot j of B; which k index a slot
// carries is a free choice as long as A and B agree.  Two orders are used:
//   * accumulator order, slot j of lane half h <-> k = 8*(j/4) + 4*h + (j%4)
//     (within a 16-block): the row order of an accumulator, so registers
//     8*kb .. 8*kb+7 of a 32x32 accumulator are the operand of k-block kb of a
//     following product that contracts over the accumulator's rows.  Scores
//     never leave registers on their way to P*V, nor the GLA state on its way
//     to Q~ S.  LDS operands paired with them come from row_operand_acc or,
//     contracting down the rows of a tile, from tr_operand (transpose reads);
//   * contiguous order, slot j <-> k = 8*h + j: row_operand, for products
//     whose two operands both come from row-major tiles or global rows.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lz {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int WAVE = 64;
constexpr float TINY = 1.1754943508222875e-38f;   // FLT_MIN, the reference's clamp
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float NEG_INF = -__builtin_huge_valf();

__device__ __forceinline__ f32x16 mfma(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Row (M index) held by accumulator register r in lane half h.
__host__ __device__ __forceinline__ constexpr int acc_row(int r, int h) {
  return ((r >> 2) << 3) + (h << 2) + (r & 3);
}

__device__ __forceinline__ float fexp(float x) { return __builtin_amdgcn_exp2f(x * LOG2E); }
__device__ __forceinline__ float flog(float x) { return __builtin_amdgcn_logf(x) * LN2; }

__device__ __forceinline__ bf16 to_bf16(float x) { return static_cast<bf16>(x); }
__device__ __forceinline__ float to_f32(bf16 x) { return static_cast<float>(x); }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

__device__ __forceinline__ bf16x8 zero_bf8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = to_bf16(0.f);
  return z;
}

// Registers 8*kb .. 8*kb+7 of an accumulator as a bf16 operand.
__device__ __forceinline__ bf16x8 acc_operand(const f32x16& acc, int kb) {
  bf16x8 o;
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = to_bf16(acc[8 * kb + j]);
  return o;
}

// Elements [c, c+4) of row `row` of a row-major [nrows x ncols] bf16 matrix,
// zero outside it.  Vector path when the row pitch keeps 8-byte alignment.
__device__ __forceinline__ bf16x4 load4(const bf16* __restrict__ p, int row, int c,
                                        int nrows, int ncols) {
  bf16x4 out;
  if (row < nrows && c + 3 < ncols && (ncols & 3) == 0) {
    out = *reinterpret_cast<const bf16x4*>(p + (size_t)row * ncols + c);
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      out[e] = (row < nrows && c + e < ncols) ? p[(size_t)row * ncols + c + e] : to_bf16(0.f);
  }
  return out;
}

// Store 4 consecutive fp32 values as OutT (bf16 or float) at [row][c..c+4),
// clipped to ncols.
template <typename OutT>
__device__ __forceinline__ void store4(OutT* __restrict__ p, int row, int c, int ncols,
                                       float a, float b, float cc, float d) {
  float v[4] = {a, b, cc, d};
  OutT* q = p + (size_t)row * ncols + c;
  if (c + 3 < ncols && (ncols & 3) == 0) {
    if constexpr (sizeof(OutT) == 2) {
      bf16x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = to_bf16(v[e]);
      *reinterpret_cast<bf16x4*>(q) = o;
    } else {
      f32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = v[e];
      *reinterpret_cast<f32x4*>(q) = o;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (c + e < ncols) {
        if constexpr (sizeof(OutT) == 2) q[e] = to_bf16(v[e]);
        else q[e] = v[e];
      }
  }
}

// Raise kernel Kern's dynamic-LDS limit to `bytes`, once per process: the
// first launch of each kernel instantiation makes the runtime call (a
// function-local static, initialised thread-safely), later launches reuse its
// status.  Every instantiation asks for one fixed size, its LDS layout's.
template <auto Kern>
hipError_t ensure_lds(int bytes) {
  static const hipError_t status = hipFuncSetAttribute(
      reinterpret_cast<const void*>(Kern), hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  return status;
}

// Row pitch (elements) of a row-major bf16 LDS tile with x columns.  Rows are
// read as 16-byte MFMA operands (8 lanes per LDS cycle) and, by the transpose
// reads, as 4 rows x 32 bytes per 16-lane group; a pitch of 36 or 72 dwords
// (mod 64 banks) keeps both conflict-free.  x + 8 gives 36 for x = 64,
// x + 16 gives 72 for x = 128 (8 for x = 256, 24 for x = 32).
__host__ __device__ constexpr int lds_pitch(int x) { return x + (x == 64 ? 8 : 16); }

// Exchange with the other half of the wave (lane ^ 32).
__device__ __forceinline__ float xhalf(float x) { return __shfl_xor(x, 32); }

// ---------------------------------------------------------------------------
// LDS transpose reads (gfx950 ds_read_b64_tr_b16).
//
// Within each group of 16 lanes, lane i receives 16-bit element i%4 of the
// 8 bytes addressed by lanes 4e + i/4 of its group, as its element e.  So if
// the 16 lanes of a group address a block of 4 rows x 16 consecutive columns
// of a row-major bf16 tile (lane 4e+q -> row e, columns 4q..4q+3), lane i
// receives column i of those 4 rows: a column read, which is what an MFMA
// operand whose k index runs down the rows of the tile needs.
// ---------------------------------------------------------------------------
typedef short short4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x4 lds_read_tr(const bf16* p) {
  typedef __attribute__((address_space(3))) short4v* lds_ptr;
  const short4v r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_ptr)(const_cast<bf16*>(p)));
  return __builtin_bit_cast(bf16x4, r);
}

// MFMA operand (A or B) whose 16 k-values run down the rows of a row-major
// bf16 LDS tile with `pitch` elements per row: lane l gets column
// col0 + l%32 at rows row0 + 4h + {0..3} (slots 0-3) and row0 + 8 + 4h + {0..3}
// (slots 4-7), h = l/32 -- the accumulator row order of acc_row(), so the
// operand pairs with accumulator-sourced operands.  col0 % 4 == 0 and
// pitch % 4 == 0 keep every lane address 8-byte aligned.
__device__ __forceinline__ bf16x8 tr_operand(const bf16* tile, int pitch, int row0, int col0,
                                             int lane) {
  const int g = lane >> 4, s = lane & 15;
  const bf16* p = tile + (row0 + 4 * (g >> 1) + (s >> 2)) * pitch + col0 + 16 * (g & 1) + 4 * (s & 3);
  const bf16x4 lo = lds_read_tr(p);
  const bf16x4 hi = lds_read_tr(p + 8 * pitch);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// MFMA operand whose 16 k-values run along row `row` of a row-major tile, in
// accumulator row order: columns col0 + 4h + {0..3} and col0 + 8 + 4h + {0..3}.
__device__ __forceinline__ bf16x8 row_operand_acc(const bf16* tile, int pitch, int row, int col0,
                                                  int h) {
  const bf16* p = tile + row * pitch + col0 + 4 * h;
  const bf16x4 lo = *reinterpret_cast<const bf16x4*>(p);
  const bf16x4 hi = *reinterpret_cast<const bf16x4*>(p + 8);
  return bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// MFMA operand whose 16 k-values are the contiguous columns col0 + 8h + {0..7}
// of row `row` (for products whose two operands both come from row-major tiles).
__device__ __forceinline__ bf16x8 row_operand(const bf16* tile, int pitch, int row, int col0,
                                              int h) {
  return *reinterpret_cast<const bf16x8*>(tile + row * pitch + col0 + 8 * h);
}

// 16-byte global load of columns [c, c+8) of row `row` of a row-major
// [nrows x ncols] bf16 matrix, zero outside it.  `vec` (ncols % 8 == 0)
// selects the single vector load; otherwise elements are loaded one by one.
__device__ __forceinline__ uint4 gload8(const bf16* __restrict__ base, int row, int c, int nrows,
                                        int ncols, bool vec) {
  if (row >= nrows) return make_uint4(0, 0, 0, 0);
  const bf16* p = base + (size_t)row * ncols + c;
  if (vec) {
    if (c < ncols) return *reinterpret_cast<const uint4*>(p);
    return make_uint4(0, 0, 0, 0);
  }
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (c + e < ncols) ? p[e] : to_bf16(0.f);
  return __builtin_bit_cast(uint4, v);
}

__device__ __forceinline__ bf16x8 scale8(const bf16x8& x, float s) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = to_bf16(to_f32(x[e]) * s);
  return o;
}

// x[j] * s[j] for the 8 slots, rounded to bf16.
__device__ __forceinline__ bf16x8 scale8v(const bf16x8& x, const f32x4& s_lo, const f32x4& s_hi) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[e] = to_bf16(to_f32(x[e]) * s_lo[e]);
    o[4 + e] = to_bf16(to_f32(x[4 + e]) * s_hi[e]);
  }
  return o;
}

}  // namespace lz
