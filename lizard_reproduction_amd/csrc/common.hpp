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
//   * contiguous order, slot j <-> k = 8*h + j: row_operand (one 16-byte
//     read) and tr_operand_c, for products whose two operands both come from
//     LDS tiles or global rows.  Where neither operand is an accumulator this
//     order is the one to use: at the row pitches used here (72, 152, 280
//     elements) the two 8-byte reads of row_operand_acc fall on the same
//     banks for rows r and r + 16, and ran at a third of the 16-byte read's
//     rate (64 against ~190 bytes per clock per CU, measured on gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

namespace lz {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// Gate mode of the GLA kernels (the C ABI's gate_mode): bit 0, one gate per
// head ([B, H, L]) rather than per token ([B, L]); bit 1, the buffer holds the
// gate logit z and log_gamma = logsigmoid(z) is formed where it is read (the
// layer's F.logsigmoid, src/lizard_attention.py:92), and the gate gradient
// written is d/dz = d log_gamma * sigmoid(-z).
constexpr int GATE_PER_HEAD = 1, GATE_LOGIT = 2, GATE_NO_REUSE = 4;

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
// 1 / max(den, FLT_MIN) by the hardware reciprocal, the output scale of the
// forward walks: within 1 ulp of fp32, far below the bf16 rounding of y that
// follows, where an IEEE division costs ten VALU instructions more
__device__ __forceinline__ float recip_den(float den) {
  return __builtin_amdgcn_rcpf(fmaxf(den, TINY));
}
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

// Raise kernel Kern's dynamic-LDS limit to `bytes` on the current device,
// once per device: the first launch of each kernel instantiation on a device
// makes the runtime call (under a per-device std::call_once), later launches
// reuse its status.  Every instantiation asks for one fixed size, its LDS
// layout's.  Devices past the table's size make the call on every launch.
constexpr int LDS_ATTR_DEVICES = 64;
template <auto Kern>
hipError_t ensure_lds(int bytes) {
  auto set = [bytes] {
    return hipFuncSetAttribute(reinterpret_cast<const void*>(Kern),
                               hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  };
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  if (dev < 0 || dev >= LDS_ATTR_DEVICES) return set();
  static std::once_flag once[LDS_ATTR_DEVICES];
  static hipError_t status[LDS_ATTR_DEVICES];
  std::call_once(once[dev], [&] { status[dev] = set(); });
  return status[dev];
}

// A kernel instantiation as a type, for launch helpers that pick one of
// several at run time and need it as a template argument (ensure_lds).
template <auto Kern>
struct KernTag {
  static constexpr auto value = Kern;
};

// Row pitch (elements) of a row-major bf16 LDS tile with x columns.  Measured
// bank-conflict cycles per instruction on gfx950 (64 banks; rocprofv3
// SQ_LDS_BANK_CONFLICT over a probe of each access pattern):
//   pitch (dwords mod 64)   16-byte rows   transpose reads   8-byte rows (acc order)
//   8  (x=128: 144)         3.9            2.0               23.5
//   12 (x=128: 152)         0              2.0               7.8
//   36 (x=64: 72)           0              2.0               7.8
// So x + 24 for x >= 128 (12 mod 64, 280 for x = 256 likewise), x + 8 for 64.
__host__ __device__ constexpr int lds_pitch(int x) {
  return x + (x == 64 ? 8 : (x >= 128 ? 24 : 16));
}

// Compute units and XCDs of the current HIP device, read once per device from
// hipDeviceAttributeMultiprocessorCount and hipDeviceAttributeNumberOfXccs.
// A whole MI355X shows 256 CUs over 8 XCDs; a partitioned one (CPX, say)
// shows each HIP device its share.  Host-only queries made without a usable
// device (workspace sizes on a machine with no GPU) get the whole chip's.
struct DevGeom {
  int cus, xcds;
};
constexpr DevGeom MI355X_GEOM = {256, 8};

inline DevGeom device_geom() {
  constexpr int MAXDEV = 64;
  static std::once_flag once[MAXDEV];
  static DevGeom geom[MAXDEV];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return MI355X_GEOM;
  std::call_once(once[dev], [dev] {
    int cus = 0, xcds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = MI355X_GEOM.cus;
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess ||
        xcds <= 0 || xcds > cus)
      xcds = 1;
    geom[dev] = DevGeom{cus, xcds};
  });
  return geom[dev];
}

// Workgroups are dispatched round-robin over the device's X XCDs (each with
// its own L2): workgroup i runs on XCD i % X.  xcd_block maps workgroup i to
// a logical block so that each XCD takes a contiguous range of `per` logical
// blocks: neighbouring logical blocks (the query heads of one kv head, the
// row blocks of one (b, h)) share an L2.  Launch xcd_grid(total, X)
// workgroups and skip logical blocks past `total`.
__host__ __device__ constexpr int xcd_grid(int total, int X) { return X * ((total + X - 1) / X); }
__device__ __forceinline__ int xcd_block(int i, int per, int X) {
  return (i % X) * per + i / X;
}

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

// tr_operand with the tile's rows scaled by scale[row] and rounded to bf16
// in registers: lane l's slots hold rows row0 + 4h + {0..3} and
// row0 + 8 + 4h + {0..3}, so their scales are two 16-byte reads (row0 % 4 == 0
// and a 16-byte aligned `scale` keep them aligned).
__device__ __forceinline__ bf16x8 tr_operand_scaled(const bf16* tile, int pitch, int row0,
                                                    int col0, int lane, const float* scale) {
  const bf16x8 x = tr_operand(tile, pitch, row0, col0, lane);
  const int h = lane >> 5;
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(scale + row0 + 4 * h);
  const f32x4 s1 = *reinterpret_cast<const f32x4*>(scale + row0 + 8 + 4 * h);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    o[e] = to_bf16(to_f32(x[e]) * s0[e]);
    o[4 + e] = to_bf16(to_f32(x[4 + e]) * s1[e]);
  }
  return o;
}

// acc + sum_{k < K} A(k) B(k) on the MFMA as a software pipeline: the
// operands of product k + P are read (from LDS) before product k issues.
// Written product by product, the compiler gives the operands one register
// set and waits for each read right before its MFMA, so the reads' latency
// adds up along the chain; the scheduling fence after each batch of reads
// keeps them ahead (only VALU and SALU work may move across it).
template <int K, int P, class FA, class FB>
__device__ __forceinline__ f32x16 mfma_chain(f32x16 acc, FA a_op, FB b_op) {
  static_assert(P >= 1 && P <= 3, "pipeline depth");
  bf16x8 a[P + 1], b[P + 1];
#pragma unroll
  for (int k = 0; k < P && k < K; ++k) {
    a[k] = a_op(k);
    b[k] = b_op(k);
  }
#pragma unroll
  for (int k = 0; k < K; ++k) {
    if (k + P < K) {
      a[(k + P) % (P + 1)] = a_op(k + P);
      b[(k + P) % (P + 1)] = b_op(k + P);
    }
    __builtin_amdgcn_sched_barrier(0x0006);
    acc = mfma(a[k % (P + 1)], b[k % (P + 1)], acc);
  }
  return acc;
}

// The same k-values as tr_operand in contiguous order (slot j <-> row
// row0 + 8h + j), to pair with row_operand.
__device__ __forceinline__ bf16x8 tr_operand_c(const bf16* tile, int pitch, int row0, int col0,
                                               int lane) {
  const int g = lane >> 4, s = lane & 15;
  const bf16* p = tile + (row0 + 8 * (g >> 1) + (s >> 2)) * pitch + col0 + 16 * (g & 1) + 4 * (s & 3);
  const bf16x4 lo = lds_read_tr(p);
  const bf16x4 hi = lds_read_tr(p + 4 * pitch);
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

// Buffer resources.  A resource covers [base, base + bytes) of global memory;
// a buffer load at a byte offset at or past `bytes` returns zeros and a
// buffer store there is dropped (the hardware's range check), so tile edges
// cost no branches.  Per-lane branches around loads are what this avoids: the
// compiler waits for each such load to land before issuing the next.  Every
// resource here spans one (batch, head) slab or one tensor of under 2 GiB
// (the host entry points check), so OOB is past the end of all of them.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t OOB = 0x80000000u;
constexpr int RSRC_WORD3 = 0x00020000;   // gfx9 dword 3: 32-bit data format, no swizzle

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, size_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)(uint32_t)(bytes < OOB ? bytes : OOB), RSRC_WORD3);
}

// AUX: the load's cache policy (LOAD_NT: nontemporal, for data that nothing
// reads again soon)
constexpr int LOAD_NT = 2;
template <int AUX = 0>
__device__ __forceinline__ uint4 bload16(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX));
}

__device__ __forceinline__ float bload_f32(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
}

// Columns [c, c+8) of row `row` of a row-major [nrows x ncols] bf16 matrix
// behind resource r, zero outside it (rows < 0 or >= nrows included).
// Vector form (ncols % 8 == 0): an item is wholly inside or outside a row.
template <int AUX = 0>
__device__ __forceinline__ uint4 bload8_vec(rsrc_t r, int row, int c, int ncols) {
  return bload16<AUX>(r, (row >= 0 && c < ncols) ? (uint32_t)(row * ncols + c) * 2u : OOB);
}

// Element form for any ncols: eight 2-byte loads.
__device__ __forceinline__ uint4 bload8_elem(rsrc_t r, int row, int c, int ncols) {
  bf16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const uint32_t off = (row >= 0 && c + e < ncols) ? (uint32_t)(row * ncols + c + e) * 2u : OOB;
    v[e] = __builtin_bit_cast(bf16, __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0));
  }
  return __builtin_bit_cast(uint4, v);
}

// One 8-column item; `vec` (ncols % 8 == 0, uniform) picks the vector form.
__device__ __forceinline__ uint4 gload8(const bf16* __restrict__ base, int row, int c, int nrows,
                                        int ncols, bool vec) {
  const rsrc_t r = make_rsrc(base, (size_t)nrows * ncols * 2);
  return vec ? bload8_vec(r, row, c, ncols) : bload8_elem(r, row, c, ncols);
}

// Row `row`, columns c0 .. c0+31 of a row-major [nrows x ncols] bf16 matrix
// behind r, from one column of a 32x32 fp32 accumulator tile (lane l holds
// tile column l % 32, register k the tile row acc_row(k, h), which is the
// matrix column c0 + acc_row(k, h)), times `scale`; rows past nrows are
// dropped.  A permlane32 swap between the two lane halves first gives half h
// the runs c0 + 16 j + 8 h + {0..7} (j = 0, 1), so each lane writes two
// 16-byte pieces (vec: ncols % 8 == 0) rather than four 8-byte ones.
template <int AUX = 0>
__device__ __forceinline__ void store_acc_row_bf16(rsrc_t r, int row, int c0, int ncols, bool vec,
                                                   const f32x16& o, float scale, int h) {
  uint32_t w[8];   // w[2g], w[2g+1]: rows 8g + 4h + {0..3} of the tile, as bf16 pairs
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const bf16x4 p = {to_bf16(o[4 * g] * scale), to_bf16(o[4 * g + 1] * scale),
                      to_bf16(o[4 * g + 2] * scale), to_bf16(o[4 * g + 3] * scale)};
    const uint2 u = __builtin_bit_cast(uint2, p);
    w[2 * g] = u.x;
    w[2 * g + 1] = u.y;
  }
  // lanes 32..63 of w[4j + k] <-> lanes 0..31 of w[4j + 2 + k]
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const auto sw = __builtin_amdgcn_permlane32_swap(w[4 * j + k], w[4 * j + 2 + k], false, false);
      w[4 * j + k] = sw[0];
      w[4 * j + 2 + k] = sw[1];
    }
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = c0 + 16 * j + 8 * h;
    if (vec) {
      const u32x4 v = {w[4 * j], w[4 * j + 1], w[4 * j + 2], w[4 * j + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(
          v, r, (row >= 0 && col < ncols) ? (uint32_t)(row * ncols + col) * 2u : OOB, 0, AUX);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint16_t x = (uint16_t)(w[4 * j + (e >> 1)] >> (16 * (e & 1)));
        __builtin_amdgcn_raw_buffer_store_b16(
            x, r, (row >= 0 && col + e < ncols) ? (uint32_t)(row * ncols + col + e) * 2u : OOB, 0,
            AUX);
      }
    }
  }
}

// The same row of a [nrows x ncols] OutT matrix at base: bf16 through
// store_acc_row_bf16 (vec: ncols % 8 == 0); fp32 as four 16-byte stores per
// lane (already whole 16-byte pieces).  Every lane of the wave must take part
// (the bf16 form swaps registers between lane halves); rows below 0 or at or
// past nrows are skipped (bf16: dropped by the buffer range check).
template <typename OutT>
__device__ __forceinline__ void store_acc_row(OutT* __restrict__ base, int row, int c0, int nrows,
                                              int ncols, bool vec, const f32x16& g, float scale,
                                              int h) {
  if constexpr (sizeof(OutT) == 2) {
    store_acc_row_bf16(make_rsrc(base, (size_t)nrows * ncols * 2), row, c0, ncols, vec, g, scale,
                       h);
  } else {
    if (row >= 0 && row < nrows) {
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4)
        store4<OutT>(base, row, c0 + 8 * g4 + 4 * h, ncols, g[4 * g4] * scale,
                     g[4 * g4 + 1] * scale, g[4 * g4 + 2] * scale, g[4 * g4 + 3] * scale);
    }
  }
}

// Items idx = threadIdx.x + NT i (i < N, idx < ITEMS) of a [rows x KP/8]
// grid of 8-column items starting at row r0: item idx covers row
// r0 + idx / (KP/8), columns 8 (idx % (KP/8)).  The uniform `vec` test sits
// outside the unrolled loop, so the vector form is straight-line loads.
template <int KP, int NT, int N, int ITEMS, int AUX = 0>
__device__ __forceinline__ void load_items(uint4 (&reg)[N], const bf16* __restrict__ base, int r0,
                                           int nrows, int ncols, bool vec) {
  constexpr int K8 = KP / 8;
  const rsrc_t r = make_rsrc(base, (size_t)nrows * ncols * 2);
  if (vec) {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = threadIdx.x + NT * i;
      if (ITEMS % NT == 0 || idx < ITEMS)
        reg[i] = bload8_vec<AUX>(r, r0 + idx / K8, (idx % K8) * 8, ncols);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int idx = threadIdx.x + NT * i;
      if (ITEMS % NT == 0 || idx < ITEMS)
        reg[i] = bload8_elem(r, r0 + idx / K8, (idx % K8) * 8, ncols);
    }
  }
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
