// Split-KV decode attention for rows with few query vectors per KV head
// (G * count <= 8): the q_len = 1 decode step and short appended chunks.
//
// Replaces, for those rows, the ATen FlashAttention-2 call of
// compiler/common/kernels/attention.cpp:66-72 / :116-117.  Math: for every
// query vector j of KV head h in row r,
//   out_j = sum_t softmax_t(scale * q_j . k_t) v_t  over keys t <= L - count + i_j
// (lower-right causal), fp32 scores / softmax / accumulation, bf16 in and out.
//
// Work item = (row, kv head, chunk of TOK_ITEM keys).  The chunk's K and V are
// read exactly once from HBM and shared by the G grouped query heads.  A
// 256-thread block = 4 waves; LPT = D/8 lanes hold one key row (16 bytes per
// lane -> one 128-bit load), so a wave instruction reads TPW = 64/LPT whole
// rows = 1 KB contiguous.  Each lane issues U loads of K then U of V before
// any arithmetic, giving 2*U*16 B in flight per lane (128 KB per block at D=128).
//   phase 1  scores: bf16 dot2 against the lane's 8 query features, reduced
//            over the LPT lanes with DPP; stored to LDS.
//   phase 2  per query vector: chunk max, p = exp2(s*scale*log2e - m), sum.
//   phase 3  o += p * v from the registers loaded in the prologue; reduced over
//            token slots (shuffles) and waves (LDS).
// With one chunk the block writes normalised bf16 output; otherwise it writes
// an fp32 partial record (o, m, l) that finalize.hip merges in a fixed order.
// The schedule depends only on the lengths, so results are deterministic and
// a row's output never depends on another row's data.
#include "device_common.h"
#include "kernel_args.h"

namespace xattn {

template <int DP, int QR, int U>
struct DecodeShape {
  static constexpr int LPT = DP / 8;        // lanes per key row
  static constexpr int TPW = 64 / LPT;      // key rows per wave instruction
  static constexpr int TOK_WAVE = TPW * U;  // keys per wave per item
  static constexpr int TOK_ITEM = 4 * TOK_WAVE;
};

template <int DP, int QR, int U>
__global__ void __launch_bounds__(256) decode_kernel(const AttnArgs a) {
  using S = DecodeShape<DP, QR, U>;
  constexpr int LPT = S::LPT, TPW = S::TPW, TOK_WAVE = S::TOK_WAVE, TOK_ITEM = S::TOK_ITEM;
  __shared__ float sc[QR][TOK_ITEM];
  __shared__ float red[4][QR][DP];
  __shared__ float stat_m[QR], stat_l[QR];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int slot = lane / LPT, dc = lane % LPT;

  const int item = blockIdx.x;
  const RowSched rs = a.rows[find_row(a.rows, a.nrows, item)];
  const int local = item - rs.item_begin;
  const int h = local / rs.nsplit, split = local - h * rs.nsplit;
  const int b = rs.batch, L = rs.length, cnt = rs.count, G = a.G;
  const int qrows = cnt * G;
  const int t0 = split * TOK_ITEM;
  const int t1 = min(L, t0 + TOK_ITEM);
  const bool dact = dc * 8 < a.D;

  // Query features of this lane's 8-wide slice, for every query vector j = i*G + g.
  u32x4 qv[QR];
#pragma unroll
  for (int j = 0; j < QR; ++j) {
    qv[j] = u32x4{0, 0, 0, 0};
    if (j < qrows && dact) {
      const int g = j % G, i = j / G;
      qv[j] = load16(a.q.p + b * a.q.sb + (int64_t)(h * G + g) * a.q.sh + (int64_t)i * a.q.st + dc * 8);
    }
  }

  // Issue every K and V load of this lane up front.  Keys >= t1 are never read.
  const uint16_t *kbase = a.k.p + b * a.k.sb + (int64_t)h * a.k.sh + dc * 8;
  const uint16_t *vbase = a.v.p + b * a.v.sb + (int64_t)h * a.v.sh + dc * 8;
  const int wt0 = t0 + wave * TOK_WAVE + slot;
  u32x4 kr[U], vr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tok = wt0 + u * TPW;
    kr[u] = (tok < t1 && dact) ? load16(kbase + (int64_t)tok * a.k.st) : u32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tok = wt0 + u * TPW;
    vr[u] = (tok < t1 && dact) ? load16(vbase + (int64_t)tok * a.v.st) : u32x4{0, 0, 0, 0};
  }

  // Phase 1: raw scores q_j . k_t.
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tok = wt0 + u * TPW;
#pragma unroll
    for (int j = 0; j < QR; ++j) {
      float d = group_sum<LPT>(dot8_bf16(kr[u], qv[j], 0.0f));
      if (dc == 0 && tok < t1) sc[j][tok - t0] = d;
    }
  }
  __syncthreads();

  // Phase 2: chunk softmax statistics, one wave per query vector.
  const int n = t1 - t0;
  for (int j = wave; j < QR; j += 4) {
    if (j >= qrows) continue;
    const int lim = L - cnt + j / G;  // last visible key of this query
    float mx = -INFINITY;
    for (int t = lane; t < n; t += 64)
      if (t0 + t <= lim) mx = fmaxf(mx, sc[j][t]);
    mx = wave_max(mx);
    const float ms = mx * a.scale_log2;
    float sum = 0.0f;
    for (int t = lane; t < n; t += 64) {
      const float p = (t0 + t <= lim && mx != -INFINITY) ? fast_exp2(fmaf(sc[j][t], a.scale_log2, -ms)) : 0.0f;
      sc[j][t] = p;
      sum += p;
    }
    sum = wave_sum(sum);
    if (lane == 0) {
      stat_m[j] = ms;
      stat_l[j] = sum;
    }
  }
  __syncthreads();

  // Phase 3: o_j += p_jt * v_t over this lane's keys.
  float acc[QR][8];
#pragma unroll
  for (int j = 0; j < QR; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[j][e] = 0.0f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int tok = wt0 + u * TPW;
    if (tok < t1) {
      const u32x4 w = vr[u];
      const float v8[8] = {bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y),
                           bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
#pragma unroll
      for (int j = 0; j < QR; ++j) {
        const float p = sc[j][tok - t0];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = fmaf(p, v8[e], acc[j][e]);
      }
    }
  }
  // Reduce over the TPW token slots of the wave (lanes dc, dc+LPT, ...).
#pragma unroll
  for (int j = 0; j < QR; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = acc[j][e];
#pragma unroll
      for (int m = LPT; m < 64; m <<= 1) x += __shfl_xor(x, m);
      acc[j][e] = x;
    }
  if (slot == 0 && dact) {
#pragma unroll
    for (int j = 0; j < QR; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[wave][j][dc * 8 + e] = acc[j][e];
  }
  __syncthreads();

  // Combine the 4 waves; write output or a partial record.
  for (int idx = tid; idx < QR * DP; idx += 256) {
    const int j = idx / DP, d = idx % DP;
    if (j >= qrows || d >= a.D) continue;
    const float o = (red[0][j][d] + red[1][j][d]) + (red[2][j][d] + red[3][j][d]);
    if (rs.nsplit == 1) {
      const int g = j % G, i = j / G;
      uint16_t *dst = a.out + b * a.o_sb + (int64_t)(h * G + g) * a.o_sh + (int64_t)i * a.o_st;
      dst[d] = (uint16_t)f32_to_bf16_bits(o / stat_l[j]);
    } else {
      const int64_t rec = rs.rec_begin + ((int64_t)h * rs.nsplit + split) * qrows + j;
      a.part_o[rec * a.D + d] = o;
      if (d == 0) {
        a.part_ml[2 * rec] = stat_m[j];
        a.part_ml[2 * rec + 1] = stat_l[j];
      }
    }
  }
}

int decode_tokens_per_item(int dp, int qr) {
  const int u = qr <= 2 ? 16 : (qr <= 4 ? 8 : 4);
  return 4 * (64 / (dp / 8)) * u;
}

template <int DP, int QR>
static hipError_t launch_decode_q(const AttnArgs &a, int items, hipStream_t stream) {
  constexpr int U = QR <= 2 ? 16 : (QR <= 4 ? 8 : 4);
  hipLaunchKernelGGL((decode_kernel<DP, QR, U>), dim3(items), dim3(256), 0, stream, a);
  return hipGetLastError();
}

template <int DP>
static hipError_t launch_decode_d(const AttnArgs &a, int qr, int items, hipStream_t stream) {
  switch (qr) {
    case 1: return launch_decode_q<DP, 1>(a, items, stream);
    case 2: return launch_decode_q<DP, 2>(a, items, stream);
    case 4: return launch_decode_q<DP, 4>(a, items, stream);
    default: return launch_decode_q<DP, 8>(a, items, stream);
  }
}

hipError_t launch_decode(const AttnArgs &a, int dp, int qr, int items, hipStream_t stream) {
  switch (dp) {
    case 64: return launch_decode_d<64>(a, qr, items, stream);
    case 128: return launch_decode_d<128>(a, qr, items, stream);
    default: return launch_decode_d<256>(a, qr, items, stream);
  }
}

}  // namespace xattn
