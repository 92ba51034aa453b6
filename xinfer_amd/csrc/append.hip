// In-place KV-cache append: the native replacement of the Triton op
// compiler/common/kernels/kv_cache.py:8-42 (launch :57-72).
//
// cache[r, h, positions[r, t], :] = new[r, h, t, :] for t < count_r, where
// count_r = cu_query[r+1] - cu_query[r].  Pure bf16 bit copies (bit-exact);
// positions of padded tokens (t >= count_r) are never dereferenced, as in
// kv_cache.py:36-39.  Unlike the Triton kernel, a position outside [0, C) is
// skipped rather than written out of bounds.
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
  const int row = blockIdx.z, head = blockIdx.y;
  const int per_token = kVector ? a.D / 8 : a.D;  // work units per token
  const int64_t unit = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int token = (int)(unit / per_token), part = (int)(unit % per_token);
  if (token >= a.T) return;
  // The new key/value rows are loaded together with the row's count (they lie
  // inside the [B, H, T, D] inputs for every token < T); the position is read
  // only for real tokens, so the copy takes two dependent memory round trips.
  const uint16_t *key = a.key.p + row * a.key.sb + head * a.key.sh + token * a.key.st;
  const uint16_t *value = a.value.p + row * a.value.sb + head * a.value.sh + token * a.value.st;
  u32x4 kv[2];
  uint16_t ks = 0, vs = 0;
  if constexpr (kVector) {
    kv[0] = load16(key + part * 8);
    kv[1] = load16(value + part * 8);
  } else {
    ks = key[part * a.key_sd];
    vs = value[part * a.value_sd];
  }
  int count = a.cu_query[row + 1] - a.cu_query[row];
  count = count < 0 ? 0 : (count > a.T ? a.T : count);
  // Keeps the key/value loads ahead of the branches below (the compiler would
  // otherwise sink them after the position load).
  if constexpr (kVector) asm volatile("" ::"v"(kv[0]), "v"(kv[1]));
  else asm volatile("" ::"v"(ks), "v"(vs));
  if (token >= count) return;  // padded token: its position is never loaded
  const int64_t pos = a.positions[row * a.pos_sb + token * a.pos_st];
  if (pos < 0 || pos >= a.C) return;
  const int64_t dst = (((int64_t)row * a.H + head) * a.C + pos) * a.D;
  if constexpr (kVector) {
    store16(a.cache_key + dst + part * 8, kv[0]);
    store16(a.cache_value + dst + part * 8, kv[1]);
  } else {
    a.cache_key[dst + part] = ks;
    a.cache_value[dst + part] = vs;
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
