// Singleton projection y[n] = sum_k W[n, k] x[k] (F.linear of one input row,
// no bias), fp32 accumulation, bf16 or fp32 in and out.
//
// Replaces the Triton op compiler/common/kernels/projection_gemv.py:10-62
// (xinfer::projection_gemv), used for the decoder's singleton projections.
// The weight is read once from HBM, so the kernel is bound by HBM bandwidth:
// n*k*sizeof(T) bytes per call.
//
// A wave reduces one row slice of KC = k / KS elements (KS slices per row,
// more when there are few rows, so that enough waves stream the weight); a
// 256-thread block is 4 waves: 4 rows (KS = 1), 2 rows x 2 slices (KS = 2)
// or 1 row x 4 slices (KS = 4).  Each lane loads 16 bytes of the row per
// step, fully coalesced (a wave reads 1 KB contiguous), and accumulates the
// exact fp32 products of its elements; the wave sums its lanes with DPP and
// cross-lane swaps, the block sums the slices through LDS in slice order.
// Rows or inputs that are not 16-byte aligned take a scalar path with the
// same structure.
#include "device_common.h"
#include "kernel_args.h"

namespace xattn {

template <typename T>
__device__ __forceinline__ float gemv_chunk(const T *w, const T *x, int i, float acc);

template <>
__device__ __forceinline__ float gemv_chunk<uint16_t>(const uint16_t *w, const uint16_t *x, int i, float acc) {
  const u32x4 a = load16(w + i), b = load16(x + i);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    acc = fmaf(bf16_lo(a[e]), bf16_lo(b[e]), acc);
    acc = fmaf(bf16_hi(a[e]), bf16_hi(b[e]), acc);
  }
  return acc;
}

template <>
__device__ __forceinline__ float gemv_chunk<float>(const float *w, const float *x, int i, float acc) {
  const f32x4 a = *as_global(reinterpret_cast<const f32x4 *>(w + i));
  const f32x4 b = *as_global(reinterpret_cast<const f32x4 *>(x + i));
  acc = fmaf(a.x, b.x, acc);
  acc = fmaf(a.y, b.y, acc);
  acc = fmaf(a.z, b.z, acc);
  acc = fmaf(a.w, b.w, acc);
  return acc;
}

__device__ __forceinline__ float to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ void store_out(uint16_t *p, float v) { *as_global(p) = (uint16_t)f32_to_bf16_bits(v); }
__device__ __forceinline__ void store_out(float *p, float v) { *as_global(p) = v; }

template <typename T, int KS, bool VEC>
__global__ void __launch_bounds__(256) gemv_kernel(const GemvArgs a) {
  constexpr int EPL = 16 / sizeof(T);  // elements per lane per 16-byte step
  __shared__ float part[4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * (4 / KS) + wave / KS;
  const int slice = wave % KS;
  const T *x = static_cast<const T *>(a.x);
  const T *w = static_cast<const T *>(a.weight) + row * a.k;
  // Slice bounds, whole 16-byte chunks except possibly the last slice.
  const int64_t per = (a.k + KS - 1) / KS;
  const int64_t k0 = VEC ? min<int64_t>(a.k, (per + EPL - 1) / EPL * EPL * slice) : min<int64_t>(a.k, per * slice);
  const int64_t k1 = VEC ? min<int64_t>(a.k, k0 + (per + EPL - 1) / EPL * EPL) : min<int64_t>(a.k, k0 + per);
  float acc = 0.0f;
  if (row < a.n) {
    if constexpr (VEC) {
      // Four 16-byte chunks per lane in flight per iteration, then the tail.
      int64_t i = k0 + (int64_t)lane * EPL;
      for (; i + 3 * 64 * EPL < k1; i += 4 * 64 * EPL) {
        float part4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int u = 0; u < 4; ++u) part4[u] = gemv_chunk<T>(w, x, (int)(i + u * 64 * EPL), 0.0f);
        acc += (part4[0] + part4[1]) + (part4[2] + part4[3]);
      }
      for (; i < k1; i += 64 * EPL) acc = gemv_chunk<T>(w, x, (int)i, acc);
    } else {
      for (int64_t i = k0 + lane; i < k1; i += 64) acc = fmaf(to_f32(as_global(w)[i]), to_f32(as_global(x)[i]), acc);
    }
  }
  acc = group_sum<64>(acc);
  if constexpr (KS > 1) {
    if (lane == 0) part[wave] = acc;
    __syncthreads();
    if (slice != 0 || lane != 0 || row >= a.n) return;
#pragma unroll
    for (int s = 1; s < KS; ++s) acc += part[wave + s];
  } else {
    if (lane != 0 || row >= a.n) return;
  }
  store_out(static_cast<T *>(a.out) + row, acc);
}

template <typename T, bool VEC>
static void launch_gemv_t(const GemvArgs &a, int ks, hipStream_t stream) {
  const dim3 grid((unsigned)((a.n * ks + 3) / 4));
  switch (ks) {
    case 1: hipLaunchKernelGGL((gemv_kernel<T, 1, VEC>), grid, dim3(256), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((gemv_kernel<T, 2, VEC>), grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((gemv_kernel<T, 4, VEC>), grid, dim3(256), 0, stream, a); break;
  }
}

hipError_t launch_gemv(const GemvArgs &a, bool fp32, bool vec, hipStream_t stream) {
  // Slices per row: enough waves to keep every CU streaming (about 16 per CU).
  const int ks = a.n >= 4096 ? 1 : (a.n >= 2048 ? 2 : 4);
  if (fp32) {
    if (vec) launch_gemv_t<float, true>(a, ks, stream);
    else launch_gemv_t<float, false>(a, ks, stream);
  } else {
    if (vec) launch_gemv_t<uint16_t, true>(a, ks, stream);
    else launch_gemv_t<uint16_t, false>(a, ks, stream);
  }
  return hipGetLastError();
}

}  // namespace xattn
