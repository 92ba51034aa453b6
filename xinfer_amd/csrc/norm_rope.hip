// The step before the attention operator in one launch: per-head RMSNorm of
// the projected queries and keys, rotary position embedding, the query written
// in the [B, Hq, T, D] layout the attention operators read, and the key and
// value appended to the KV cache in place.
//
// Replaces the eager sequence of compiler/qwen3/adapters/attention.py:44-51:
//   q = q_norm(q_proj(x).view(B, T, Hq, D)).transpose(1, 2)
//   k = k_norm(k_proj(x).view(B, T, Hkv, D)).transpose(1, 2)
//   v = v_proj(x).view(B, T, Hkv, D).transpose(1, 2)
//   q, k = apply_rotary_pos_emb(q, k, cos, sin)
//   append_kv_batched(k, v, positions, cu_query, cache_key, cache_value)
// with the arithmetic and bf16 rounding points of those modules
// (transformers Qwen3RMSNorm and apply_rotary_pos_emb):
//   y  = bf16(x * rsqrt(mean(x^2) + eps))        mean, rsqrt in fp32
//   xn = bf16(w * y)
//   out_i = bf16(bf16(xn_i * cos_i) + bf16(rot_i * sin_i)),
//   rot_i = -xn_{i + D/2} for i < D/2, xn_{i - D/2} otherwise.
// Products of two bf16 values are exact in fp32, so every bf16 result above is
// the rounding of the same fp32 value the eager modules round; only mean(x^2),
// a sum whose order differs between implementations, may differ in its last
// bit.
//
// One row = (token, projected head): the Hq query heads, then the Hkv key
// heads, then the Hkv value heads of each token.  LPR = D/8 lanes hold a row,
// 8 features (16 bytes) each; a 256-thread block holds 256/LPR rows.  The
// partner of lane c for the rotation is lane c ^ LPR/2 (the other half of the
// row).  A key or value row is written to the cache only for a real token
// (t < count_r) whose position lies in [0, C); query rows are written for
// every token, as the eager sequence computes them.
#include "device_common.h"
#include "kernel_args.h"

namespace xattn {

__device__ __forceinline__ float round_bf16(float x) { return __uint_as_float(f32_to_bf16_bits(x) << 16); }

template <int LPR>
__global__ void __launch_bounds__(256) norm_rope_kernel(const NormRopeArgs a) {
  constexpr int ROWS = 256 / LPR;
  const int lane_row = threadIdx.x / LPR, dc = threadIdx.x % LPR;
  const int64_t grow = (int64_t)blockIdx.x * ROWS + lane_row;
  const int per_token = a.Hq + 2 * a.Hkv;
  const int64_t token = grow / per_token;
  if (token >= (int64_t)a.B * a.T) return;  // whole rows only: LPR lanes exit together
  const int which = (int)(grow - token * per_token);
  const int b = (int)(token / a.T), t = (int)(token - (int64_t)b * a.T);
  const int kind = which < a.Hq ? 0 : (which < a.Hq + a.Hkv ? 1 : 2);  // query, key, value
  const int h = kind == 0 ? which : (kind == 1 ? which - a.Hq : which - a.Hq - a.Hkv);
  const View &src = kind == 0 ? a.q : (kind == 1 ? a.k : a.v);

  // Every load of the row in one round trip.
  const u32x4 x = load16(src.p + b * src.sb + h * src.sh + t * src.st + dc * 8);
  u32x4 w{0, 0, 0, 0}, cs{0, 0, 0, 0}, sn{0, 0, 0, 0};
  if (kind < 2) {
    w = load16((kind == 0 ? a.q_weight : a.k_weight) + dc * 8);
    cs = load16(a.cos.p + b * a.cos.sb + t * a.cos.st + dc * 8);
    sn = load16(a.sin.p + b * a.sin.sb + t * a.sin.st + dc * 8);
  }
  int32_t c0 = 0, c1 = 0;
  int64_t pos = -1;
  if (kind > 0) {
    c0 = as_global(a.cu_query)[b];
    c1 = as_global(a.cu_query)[b + 1];
    pos = as_global(a.positions)[b * a.pos_sb + t * a.pos_st];
  }

  u32x4 outw = x;
  if (kind < 2) {
    float xf[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xf[2 * e] = bf16_lo(x[e]);
      xf[2 * e + 1] = bf16_hi(x[e]);
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(xf[e], xf[e], ss);  // x^2 is exact in fp32
    ss = group_sum<LPR>(ss);
    const float inv = rsqrtf(ss / (float)(LPR * 8) + a.eps);
    float xn[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      xn[2 * e] = round_bf16(bf16_lo(w[e]) * round_bf16(xf[2 * e] * inv));
      xn[2 * e + 1] = round_bf16(bf16_hi(w[e]) * round_bf16(xf[2 * e + 1] * inv));
    }
    // The other half of the row, from the partner lane c ^ LPR/2: DPP
    // row_ror:8 within a 16-lane row (LPR = 16), the permlane16 swap (LPR =
    // 32); a shuffle through LDS for LPR = 8.
    float pn[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (LPR == 16) {
        pn[e] = dpp_move<kDppRowRor8>(xn[e]);
      } else if constexpr (LPR == 32) {
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(xn[e]), __float_as_uint(xn[e]), false, false);
        pn[e] = __uint_as_float(dc < 16 ? r[1] : r[0]);
      } else {
        pn[e] = __shfl_xor(xn[e], LPR / 2, LPR);
      }
    }
    const bool lower = dc < LPR / 2;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float o[2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = 2 * e + u;
        const float c = u ? bf16_hi(cs[e]) : bf16_lo(cs[e]);
        const float s = u ? bf16_hi(sn[e]) : bf16_lo(sn[e]);
        const float rot = lower ? -pn[i] : pn[i];
        o[u] = round_bf16(round_bf16(xn[i] * c) + round_bf16(rot * s));
      }
      outw[e] = pack_bf16x2(o[0], o[1]);
    }
  }

  if (kind == 0) {
    store16(a.q_out + ((int64_t)(b * a.Hq + h) * a.T + t) * (LPR * 8) + dc * 8, outw);
    return;
  }
  int count = c1 - c0;
  count = count < 0 ? 0 : (count > a.T ? a.T : count);
  if (t >= count || pos < 0 || pos >= a.C) return;
  uint16_t *cache = kind == 1 ? a.cache_key : a.cache_value;
  store16(cache + (((int64_t)b * a.Hkv + h) * a.C + pos) * (LPR * 8) + dc * 8, outw);
}

hipError_t launch_norm_rope(const NormRopeArgs &a, hipStream_t stream) {
  const int64_t rows = (int64_t)a.B * a.T * (a.Hq + 2 * a.Hkv);
  const int lpr = a.D / 8;
  const dim3 grid((unsigned)((rows * lpr + 255) / 256));
  switch (lpr) {
    case 8: hipLaunchKernelGGL((norm_rope_kernel<8>), grid, dim3(256), 0, stream, a); break;
    case 16: hipLaunchKernelGGL((norm_rope_kernel<16>), grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((norm_rope_kernel<32>), grid, dim3(256), 0, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace xattn
