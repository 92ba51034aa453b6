// Helpers shared by the MFMA prefill kernels (prefill.hip: head dims 64 and
// 128; prefill_d256.hip: head dim 256): the MFMA and transposing-LDS-read
// wrappers, HBM -> LDS buffer loads, wait/barrier helpers, the key range of a
// split and the LDS swizzles of K and V rows.
//
// MFMA 32x32x16 lane layout used (A: 32xK16, B: K16x32, C: 32x32):
//   A lane l: row l%32, k = 8*(l/32) + 0..7      B lane l: col l%32, same k
//   C lane l, reg r: row 8*(r/4) + 4*(l/32) + r%4, col l%32
#pragma once

#include "device_common.h"

namespace xattn {

constexpr int kTileQ = 128;  // query vectors per prefill work item

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Transposing 8-byte LDS read (ds_read_b64_tr_b16): within each 16-lane group,
// lane j supplies the address of V[k0 + j/4][d0 + 4(j%4) .. +3] and receives
// V[k0 .. k0+3][d0 + j], i.e. four consecutive keys of one feature, which is
// the A-operand layout of the PV product.
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t *p) {
  const shortx4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) shortx4 *)(p));
  return __builtin_bit_cast(u32x2, r);
}

// One 16-byte-per-lane buffer load into LDS: lane i's 16 bytes land at LDS
// byte address m0 + 16 * i.  Written as inline asm so that the compiler does
// not track these loads: it would otherwise wait for all of them before any
// transposing LDS read, which would drain the load pipeline every tile.  The
// waits for them are explicit (wait_loads_and_barrier); loads the compiler
// does track are unaffected, since extra outstanding loads only make its own
// waits stricter.
__device__ __forceinline__ void lds_load16(u32x4 rsrc, uint32_t lds_byte, uint32_t voffset, uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_byte)), "v"(voffset), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory", "m0");
}

// Buffer descriptor words for [base, base + bytes) (raw buffer, no stride;
// loads past `bytes` return zero).
__device__ __forceinline__ u32x4 buffer_words(const void *base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  return u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xffffu, bytes, 0x00020000u};
}

__device__ __forceinline__ uint32_t lds_address(const void *p) {
  return (uint32_t)(uintptr_t)(lds_void *)(p);
}

// Wait until at most N vector-memory operations of this wave are outstanding
// (loads return in issue order), then synchronise the block.  The empty asm
// keeps the compiler from moving LDS accesses across the barrier.
template <int N>
__device__ __forceinline__ void wait_loads_and_barrier() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  // s_waitcnt encoding (gfx9): vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt_hi[15:14].
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Wait for this wave's LDS accesses, then synchronise the block.
__device__ __forceinline__ void wait_lds_and_barrier() {
  __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Wait until at most N of this wave's vector-memory operations are
// outstanding and for its LDS accesses, then synchronise the block.
template <int N>
__device__ __forceinline__ void wait_loads_lds_and_barrier() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0x0 << 8));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Key range [ks0, ks1) of split `split` for a tile whose last visible key is kend-1.
template <int BN>
__device__ __forceinline__ void split_range(int kend, int nsplit, int split, int &ks0, int &ks1) {
  const int per = ((kend + nsplit - 1) / nsplit + BN - 1) / BN * BN;
  ks0 = min(kend, split * per);
  ks1 = min(kend, ks0 + per);
}

// XOR swizzles of the 16-byte chunks of a key row (chunk c of key k is stored
// at slot c ^ swz(k)).  K: a K read takes chunk c of 32 consecutive keys, so
// the 16 keys served together land in 16 different slots.  V: the 32 lanes
// one LDS pass serves (8 bytes each) read chunks 4t .. 4t+3 of 4 consecutive
// keys (k0 % 4 == 0); the swizzle moves each key's four chunks to its own
// group of four slots, i.e. its own 16 of the 64 banks.  (With D = 64 two
// rows share the banks, so keys k and k+1 already differ in bank half.)
template <int CHUNKS>
__device__ __forceinline__ int k_swizzle(int key) { return key & (CHUNKS >= 16 ? 15 : CHUNKS - 1); }
template <int CHUNKS>
__device__ __forceinline__ int v_swizzle(int key) { return CHUNKS >= 16 ? 4 * (key & 3) : 4 * ((key >> 1) & 1); }

// Zero out[b, h*G + g, t, :] for the row's padded queries t in [cnt, T) (the
// tile-0 / split-0 item of each kv head does it).
__device__ __forceinline__ void zero_padded_queries(const AttnArgs &a, int b, int h, int cnt, int G, int D, int T,
                                                    int tid, int threads) {
  const int chunks = D / 8, per = (T - cnt) * chunks;
  for (int idx = tid; idx < G * per; idx += threads) {
    const int g = idx / per, rest = idx - g * per;
    const int t = cnt + rest / chunks, ch = rest - (rest / chunks) * chunks;
    store16(a.out + b * a.o_sb + (int64_t)(h * G + g) * a.o_sh + (int64_t)t * a.o_st + ch * 8, u32x4{0, 0, 0, 0});
  }
}

}  // namespace xattn
