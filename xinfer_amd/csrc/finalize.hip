// Finalize pass of a split-KV attention call: merge the fp32 partial records
// of rows whose keys were split across work items, and write the zero output
// of padded queries (t >= count_r), which the reference produces with
// at::zeros + per-row copies (compiler/common/kernels/attention.cpp:54,73-77).
//
// One wave per output query vector (b, hq, t); a lane owns 4 features.  For a
// merged vector with partials (m_s, l_s, o_s), s = 0..S-1 (m in log2 units):
//   M = max_s m_s,  w_s = exp2(m_s - M),  out = sum_s w_s o_s / sum_s w_s l_s
// in increasing s, so the result is deterministic.  Splits that saw no visible
// key carry m = -inf and get weight 0.
#include "device_common.h"
#include "kernel_args.h"

namespace xattn {

__global__ void __launch_bounds__(256) finalize_kernel(const FinalizeArgs a) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t vec = (int64_t)blockIdx.x * 4 + wave;  // query vector within this launch
  const int64_t per_row = (int64_t)a.Hq * a.T;
  if (vec >= (int64_t)a.nrows * per_row) return;
  const int r = (int)(vec / per_row);
  const int hq = (int)((vec % per_row) / a.T);
  const int t = (int)(vec % a.T);
  const FinalizeRow fr = a.rows[r];
  const int b = a.row_base + r;
  uint16_t *dst = a.out + (((int64_t)b * a.Hq + hq) * a.T + t) * a.D;
  const int d = lane * 4;
  if (t >= fr.count) {
    if (d < a.D) *reinterpret_cast<u32x2 *>(dst + d) = u32x2{0u, 0u};
    return;
  }
  if (fr.nsplit <= 1) return;  // written directly by the attention kernel
  const int h = hq / a.G, g = hq % a.G;
  const int qrows = fr.count * a.G;
  const int j = t * a.G + g;
  const int64_t rec0 = fr.rec_begin + (int64_t)h * fr.nsplit * qrows + j;
  float m = -INFINITY;
  for (int s = 0; s < fr.nsplit; ++s) m = fmaxf(m, a.part_ml[2 * (rec0 + (int64_t)s * qrows)]);
  float l = 0.0f;
  f32x4 o = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s = 0; s < fr.nsplit; ++s) {
    const int64_t rec = rec0 + (int64_t)s * qrows;
    const float ms = a.part_ml[2 * rec];
    if (ms == -INFINITY) continue;
    const float w = fast_exp2(ms - m);
    l = fmaf(w, a.part_ml[2 * rec + 1], l);
    if (d < a.D) {
      const f32x4 ps = *reinterpret_cast<const f32x4 *>(a.part_o + rec * a.D + d);
      o.x = fmaf(w, ps.x, o.x);
      o.y = fmaf(w, ps.y, o.y);
      o.z = fmaf(w, ps.z, o.z);
      o.w = fmaf(w, ps.w, o.w);
    }
  }
  if (d < a.D) {
    const float inv = 1.0f / l;
    *reinterpret_cast<u32x2 *>(dst + d) = u32x2{pack_bf16x2(o.x * inv, o.y * inv), pack_bf16x2(o.z * inv, o.w * inv)};
  }
}

hipError_t launch_finalize(const FinalizeArgs &a, hipStream_t stream) {
  const int64_t vecs = (int64_t)a.nrows * a.Hq * a.T;
  if (vecs == 0) return hipSuccess;
  hipLaunchKernelGGL(finalize_kernel, dim3((unsigned)((vecs + 3) / 4)), dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace xattn
