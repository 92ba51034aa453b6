// Device-side helpers for the gfx950 (CDNA4) attention kernels: bf16 bit
// conversions, 16-byte vector types, DPP row reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernel_args.h"

namespace xattn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Round-to-nearest-even float -> bf16 bits (hardware conversion on gfx950).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

__device__ __forceinline__ bf16x2 as_bf16x2(uint32_t w) { return __builtin_bit_cast(bf16x2, w); }
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 w) { return __builtin_bit_cast(bf16x8, w); }

// Global-memory pointer of p.  Kernels pin their arguments in SGPRs with an
// empty asm statement (XATTN_PIN_VIEW below); a pointer that went through it
// has lost the address space the compiler inferred for kernel arguments, and
// accesses through it would become flat instructions (which also count
// against the LDS counter).  as_global() restores the global address space.
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T *as_global(T *p) {
  return (__attribute__((address_space(1))) T *)p;
}

// 16-byte global-memory load and store.
__device__ __forceinline__ u32x4 load16(const uint16_t *p) {
  return *as_global(reinterpret_cast<const u32x4 *>(p));
}
__device__ __forceinline__ void store16(uint16_t *p, u32x4 v) { *as_global(reinterpret_cast<u32x4 *>(p)) = v; }

// 4-term bf16 dot product of two 8-element bf16 vectors accumulated in fp32.
__device__ __forceinline__ float dot8_bf16(u32x4 a, u32x4 b, float acc) {
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.x), as_bf16x2(b.x), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.y), as_bf16x2(b.y), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.z), as_bf16x2(b.z), acc, false);
  acc = __builtin_amdgcn_fdot2_f32_bf16(as_bf16x2(a.w), as_bf16x2(b.w), acc, false);
  return acc;
}

// DPP lane move within a 16-lane row (gfx9 encodings).
template <int CTRL>
__device__ __forceinline__ float dpp_move(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within each 8-lane half row
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within each 16-lane row

// All-reduce over lanes {l, l ^ 16} / {l, l ^ 32} with the gfx950 permlane
// swaps.  A swap of x with itself returns x's even-row (lower-half) and
// odd-row (upper-half) copies in its two results; their sum / max is the
// reduction over the pair on every lane, in the same order on both lanes.
__device__ __forceinline__ float pair_sum16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_sum32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair_max16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_max32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
constexpr int kDppRowRor8 = 0x128;    // lane i <- lane (i + 8) mod 16 within each row
constexpr int kDppRowRor4 = 0x124;    // lane i <- lane (i + 4) mod 16 within each row

// All-reduce (sum) over aligned groups of N lanes, N in {8,16,32,64}.  Every lane
// of a group ends with the same value (each level adds a pair of equal partials).
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp_move<kDppXor1>(x);
  x += dpp_move<kDppXor2>(x);
  x += dpp_move<kDppHalfMirror>(x);
  if constexpr (N >= 16) x += dpp_move<kDppMirror>(x);
  if constexpr (N >= 32) x = pair_sum16(x);
  if constexpr (N >= 64) x += __shfl_xor(x, 32);
  return x;
}


// Reductions over the lanes l, l + S, l + 2S, ... (S = stride, a power of two
// >= 8): the key-row slots of a wave in the decode kernel.
template <int S>
__device__ __forceinline__ float slot_sum(float x) {
  if constexpr (S <= 8) x += dpp_move<kDppRowRor8>(x);
  if constexpr (S <= 16) x = pair_sum16(x);
  if constexpr (S <= 32) x = pair_sum32(x);
  return x;
}
template <int S>
__device__ __forceinline__ float slot_max(float x) {
  if constexpr (S <= 8) x = fmaxf(x, dpp_move<kDppRowRor8>(x));
  if constexpr (S <= 16) x = pair_max16(x);
  if constexpr (S <= 32) x = pair_max32(x);
  return x;
}

// Reduce-scatter of QR (2 or 4) per-lane partial dot products over aligned
// groups of N (16 or 32) lanes: lane l ends with the group's full sum for
// query l & (QR - 1).  The first log2(QR) steps halve the values each lane
// keeps (DPP xor 1, xor 2); the rest all-reduce over the lanes of one query
// with symmetric steps (xor 2 for QR = 2, rotate 8 then rotate 4 within the
// 16-lane row, the permlane16 pair), so those lanes end with equal sums.
template <int QR, int N>
__device__ __forceinline__ float rs_sum(const float (&d)[QR], int lane) {
  static_assert((QR == 2 || QR == 4) && (N == 16 || N == 32), "reduce-scatter shape");
  const bool b0 = lane & 1;
  float v;
  if constexpr (QR == 4) {
    const float k0 = b0 ? d[1] : d[0], k1 = b0 ? d[3] : d[2];
    const float s0 = b0 ? d[0] : d[1], s1 = b0 ? d[2] : d[3];
    const float n0 = k0 + dpp_move<kDppXor1>(s0), n1 = k1 + dpp_move<kDppXor1>(s1);
    const bool b1 = lane & 2;
    const float kk = b1 ? n1 : n0, ss = b1 ? n0 : n1;
    v = kk + dpp_move<kDppXor2>(ss);
  } else {
    const float k0 = b0 ? d[1] : d[0], s0 = b0 ? d[0] : d[1];
    v = k0 + dpp_move<kDppXor1>(s0);
    v += dpp_move<kDppXor2>(v);
  }
  v += dpp_move<kDppRowRor8>(v);
  v += dpp_move<kDppRowRor4>(v);
  if constexpr (N == 32) v = pair_sum16(v);
  return v;
}
// Value of query J from the lane of the quad that holds it (after rs_sum).
template <int QR, int J>
__device__ __forceinline__ float quad_query(float x) {
  constexpr int ctrl = QR == 4 ? J * 0x55 : (J == 0 ? 0xA0 : 0xF5);
  return dpp_move<ctrl>(x);
}

__device__ __forceinline__ float wave_max(float x) {
  for (int m = 32; m >= 1; m >>= 1) x = fmaxf(x, __shfl_xor(x, m));
  return x;
}
__device__ __forceinline__ float wave_sum(float x) {
  for (int m = 32; m >= 1; m >>= 1) x += __shfl_xor(x, m);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Raw buffer resource over [base, base + bytes): the 64-bit base lives in
// scalar registers and loads take a 32-bit lane offset plus a scalar offset.
// Range checking makes a load at or past `bytes` return zero without a
// memory access.  0x00020000 is the descriptor's fourth dword on the gfx9
// family (32-bit data format, no swizzle).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void *base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// Loads with cache policy sc0 (scope beyond the CU): they miss in the CU's L1
// and read the XCD's L2, i.e. data other CUs of the same XCD stored during
// this launch.
__device__ __forceinline__ u32x4 buffer_load16_l2(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, 0, 1));
}
__device__ __forceinline__ u32x2 buffer_load8_l2(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset) {
  return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(rsrc, voffset, 0, 1));
}
// Non-temporal (cache policy nt) 16-byte load, for data read exactly once.
__device__ __forceinline__ u32x4 buffer_load16_stream(__amdgpu_buffer_rsrc_t rsrc, uint32_t voffset, uint32_t soffset) {
  return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, soffset, 2));
}

// Kernel arguments reach a wave through scalar loads from the kernarg
// segment.  The compiler issues each load next to its first use and may load a
// value again at a later use, so a prologue that reads its arguments in stages
// waits one memory round trip per stage.  A kernel therefore copies the
// arguments it needs into locals and ties them all to SGPRs in ONE empty asm
// statement (separate statements are scheduling boundaries, and the loads
// would again come in stages): one round trip, and later uses read the
// registers.  These macros spell the operand lists.
#define XATTN_PIN_VIEW(v) "+s"((v).p), "+s"((v).sb), "+s"((v).sh), "+s"((v).st)
#define XATTN_PIN_ROWSCHED(r)                                                                 \
  "+s"((r).batch), "+s"((r).count), "+s"((r).length), "+s"((r).item_begin), "+s"((r).nsplit), \
      "+s"((r).ntiles), "+s"((r).rec_begin)
#define XATTN_PIN_MERGEROW(r)                                                                 \
  "+s"((r).batch), "+s"((r).count), "+s"((r).nsplit), "+s"((r).item_begin), "+s"((r).tiles), \
      "+s"((r).rec_begin)
#define XATTN_PIN_BEGINS(l)                                                                   \
  "+s"((l).begin[0]), "+s"((l).begin[1]), "+s"((l).begin[2]), "+s"((l).begin[3]),             \
      "+s"((l).begin[4]), "+s"((l).begin[5]), "+s"((l).begin[6]), "+s"((l).begin[7])

// Row lookup over a kernarg row table sorted by item_begin.  load() reads the
// first eight item_begin values and row 0 (the tables always hold kMaxRows >= 8
// rows, so the reads stay inside the arguments), to be pinned with the caller's
// other arguments (XATTN_PIN_BEGINS and the row's list); find() then needs a
// second round trip only for an item of a row other than 0, and a scan of the
// table only past eight rows.
template <typename Row>
struct RowLookup {
  static_assert(kMaxRows >= 8, "row table");
  int begin[8];
  Row first;
  __device__ __forceinline__ void load(const Row *rows) {
#pragma unroll
    for (int k = 0; k < 8; ++k) begin[k] = rows[k].item_begin;
    first = rows[0];
  }
  __device__ __forceinline__ Row find(const Row *rows, int nrows, int item) const {
    int r = 0;
#pragma unroll
    for (int k = 1; k < 8; ++k) r = (k < nrows && begin[k] <= item) ? k : r;
    for (int k = 8; k < nrows; ++k)
      if (rows[k].item_begin <= item) r = k;
    return r == 0 ? first : rows[r];
  }
};

// Cache row that holds row b's K/V under a page table (the reference's paged
// FlashAttention call, compiler/common/kernels/attention.cpp:39-40, 68-70):
// blocks[b * stride] clamped into [0, rows), so that no table can address
// outside k/v; b itself without a table.  Kernels issue the read before their
// first K/V loads (for row b) and clamp and compare it where those loads are
// awaited anyway, reissuing them only when the page differs.  The read is a
// scalar load (constant address space, block-uniform address), so waiting
// for it never waits for vector loads.
__device__ __forceinline__ int read_page(const int32_t *blocks, int64_t stride, int b) {
  if (blocks == nullptr) return b;
  typedef const __attribute__((address_space(4))) int32_t *table_ptr;
  return ((table_ptr)blocks)[(int64_t)b * stride];
}
__device__ __forceinline__ int page_in_range(int page, int rows) { return min(max(page, 0), rows - 1); }

// Row r's query count and KV length from the device offsets, clamped to the
// ranges the host validates in the default mode (see CaptureArgs in kernel_args.h).
__device__ __forceinline__ void capture_row(const CaptureArgs &c, int r, int &count, int &length) {
  const int32_t *cuq = c.offsets, *cuk = c.offsets + c.B + 1;
  count = min(max(cuq[r + 1] - cuq[r], 0), min(c.T, c.C));
  length = min(max(cuk[r + 1] - cuk[r], max(count, 1)), c.C);
}

}  // namespace xattn
