// In-place KV-cache append: the native replacement of the Triton op
// compiler/common/kernels/kv_cache.py:8-42 (launch :57-72).
//
// cache[r, h, positions[r, t], :] = new[r, h, t, :] for t < count_r, where
// count_r = cu_query[r+1] - cu_query[r].  Pure bf16 bit copies (bit-exact);
// positions of padded tokens (t >= count_r) are not used, as in
// kv_cache.py:36-39 (they are loaded with the rest, inside the [B, T] tensor).
// Unlike the Triton kernel, a position outside [0, C) is skipped rather than
// written out of bounds.
//
// Grid: x = token blocks, y = kv head, z = row.  On the vector path each lane
// moves one 16-byte chunk (8 features) of key and of value, so a 256-thread
// block copies 256*16 B of each; consecutive lanes cover consecutive chunks of
// a token row (coalesced reads and writes).
#include "device_common.h"
#include "kernel_args.h"

namespace xattn {

template <bool kVector>
__global__ void __launch_bounds__(256) append_kv_kernel(const AppendArgs a) {
  // Every argument, loaded in one round trip (see XATTN_PIN_VIEW).
  View kin = a.key, vin = a.value;
  int64_t key_sd = a.key_sd, value_sd = a.value_sd, pos_sb = a.pos_sb, pos_st = a.pos_st;
  const int64_t *positions = a.positions;
  const int32_t *cu_query = a.cu_query;
  uint16_t *cache_key = a.cache_key, *cache_value = a.cache_value;
  int H = a.H, T = a.T, D = a.D, C = a.C;
  asm volatile(""
               : XATTN_PIN_VIEW(kin), XATTN_PIN_VIEW(vin), "+s"(key_sd), "+s"(value_sd), "+s"(pos_sb), "+s"(pos_st),
                 "+s"(positions), "+s"(cu_query), "+s"(cache_key), "+s"(cache_value), "+s"(H), "+s"(T), "+s"(D),
                 "+s"(C));
  const int row = blockIdx.z, head = blockIdx.y;
  const int per_token = kVector ? D / 8 : D;  // work units per token
  const int64_t unit = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int token = (int)(unit / per_token), part = (int)(unit % per_token);
  if (token >= T) return;
  // The new key/value rows, the row's count and the token's position are
  // loaded together (one memory round trip): every token < T lies inside the
  // [B, H, T, D] inputs and the [B, T] positions.  A padded token's position
  // is loaded but never used.
  const uint16_t *key = kin.p + row * kin.sb + head * kin.sh + token * kin.st;
  const uint16_t *value = vin.p + row * vin.sb + head * vin.sh + token * vin.st;
  u32x4 kv[2];
  uint16_t ks = 0, vs = 0;
  if constexpr (kVector) {
    kv[0] = load16(key + part * 8);
    kv[1] = load16(value + part * 8);
  } else {
    ks = as_global(key)[part * key_sd];
    vs = as_global(value)[part * value_sd];
  }
  const int32_t c0 = as_global(cu_query)[row], c1 = as_global(cu_query)[row + 1];
  const int64_t pos = as_global(positions)[row * pos_sb + token * pos_st];
  // Keeps every load ahead of the branches below (the compiler would otherwise
  // sink the key/value loads after them, a second round trip).
  if constexpr (kVector) asm volatile("" ::"v"(kv[0]), "v"(kv[1]), "v"(c0), "v"(c1), "v"(pos));
  else asm volatile("" ::"v"(ks), "v"(vs), "v"(c0), "v"(c1), "v"(pos));
  int count = c1 - c0;
  count = count < 0 ? 0 : (count > T ? T : count);
  if (token >= count) return;  // padded token
  if (pos < 0 || pos >= C) return;
  const int64_t dst = (((int64_t)row * H + head) * C + pos) * D;
  if constexpr (kVector) {
    store16(cache_key + dst + part * 8, kv[0]);
    store16(cache_value + dst + part * 8, kv[1]);
  } else {
    as_global(cache_key)[dst + part] = ks;
    as_global(cache_value)[dst + part] = vs;
  }
}

hipError_t launch_append(const AppendArgs &a, bool vector, hipStream_t stream) {
  const int64_t units = (int64_t)a.T * (vector ? a.D / 8 : a.D);
  const dim3 grid((unsigned)((units + 255) / 256), (unsigned)a.H, (unsigned)a.B);
  if (vector)
    hipLaunchKernelGGL(append_kv_kernel<true>, grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(append_kv_kernel<false>, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace xattn
