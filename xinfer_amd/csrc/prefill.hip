// Chunked causal prefill attention on the gfx950 matrix cores (MFMA bf16).
//
// Replaces, for rows with more than 8 query vectors per KV head, the ATen
// FlashAttention-2 calls of compiler/common/kernels/attention.cpp:66-72 and
// :116-117.  Same math as decode.hip: lower-right causal softmax(scale*QK^T)V
// over the populated prefix, fp32 softmax state, bf16 in/out.
//
// Work item = (row, kv head, tile of 128 query vectors, KV split).  The query
// vectors of one KV head are enumerated j = i*G + g (query i, grouped head g),
// so one tile serves all G heads that share the K/V tile in LDS.
//
// The block's 4 waves each own 32 query vectors and compute the transposed
// problem with v_mfma_f32_32x32x16_bf16:
//   S^T[key, j]  = K[key, :] . Q[j, :]      A = K tile (LDS), B = Q^T (registers)
//   O^T[d, j]   += V^T[d, key] P^T[key, j]  A = V^T tile (LDS), B = P^T (from S^T)
// In this orientation a lane's accumulator column is one query vector, so the
// online-softmax max/sum are per-lane (plus one exchange with lane^32), and the
// S^T accumulator registers are already the B operand of the PV product: no
// LDS round trip for P.  K is staged row-major, V transposed ([d][key]) so the
// PV A operand is two 8-byte LDS reads.
//
// MFMA 32x32x16 lane layout used (A: 32xK16, B: K16x32, C: 32x32):
//   A lane l: row l%32, k = 8*(l/32) + 0..7      B lane l: col l%32, same k
//   C lane l, reg r: row 8*(r/4) + 4*(l/32) + r%4, col l%32
// The PV product contracts over keys; the key <-> k-slot assignment only has to
// agree between the A and B operands, and both are derived from the C layout.
#include "device_common.h"
#include "kernel_args.h"

namespace xattn {

constexpr int kTileQ = 128;  // query vectors per work item
constexpr int kBN = 64;      // keys per LDS tile

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Key range [ks0, ks1) of split `split` for a tile whose last visible key is kend-1.
__device__ __forceinline__ void split_range(int kend, int nsplit, int split, int &ks0, int &ks1) {
  const int per = ((kend + nsplit - 1) / nsplit + kBN - 1) / kBN * kBN;
  ks0 = min(kend, split * per);
  ks1 = min(kend, ks0 + per);
}

template <int DP>
__global__ void __launch_bounds__(256) prefill_kernel(const AttnArgs a) {
  constexpr int KP = DP + 8;   // K tile pitch (bf16 elements); 16-byte pad
  constexpr int VP = kBN + 8;  // V^T tile pitch
  constexpr int NDS = DP / 16; // k-steps of the QK product
  constexpr int NDT = DP / 32; // 32-row d tiles of the output
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[DP * VP];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;

  const int item = blockIdx.x;
  const RowSched rs = a.rows[find_row(a.rows, a.nrows, item)];
  const int local = item - rs.item_begin;
  const int per_head = rs.ntiles * rs.nsplit;
  const int h = local / per_head;
  const int tile = (local - h * per_head) / rs.nsplit;
  const int split = local - h * per_head - tile * rs.nsplit;
  const int b = rs.batch, L = rs.length, cnt = rs.count, G = a.G, D = a.D;
  const int qrows = cnt * G, p0 = L - cnt;

  // Key range of this tile and split.
  const int j_last = min(tile * kTileQ + kTileQ, qrows) - 1;
  const int kend = p0 + j_last / G + 1;
  int ks0, ks1;
  split_range(kend, rs.nsplit, split, ks0, ks1);

  // This lane's query vector.
  const int j = tile * kTileQ + wave * 32 + col;
  const bool jvalid = j < qrows;
  const int g = j % G, qi = j / G;
  const int lim = p0 + qi;  // last visible key
  const int jw_first = tile * kTileQ + wave * 32;
  const bool wave_active = jw_first < qrows;
  const int wave_kmax = p0 + (min(jw_first + 31, qrows - 1)) / G;  // last key any column sees
  const int wave_kmin = p0 + jw_first / G;                          // last key of the first column

  bf16x8 qf[NDS];
  {
    const uint16_t *qp = a.q.p + b * a.q.sb + (int64_t)(h * G + g) * a.q.sh + (int64_t)qi * a.q.st;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const int d = ds * 16 + half * 8;
      qf[ds] = as_bf16x8((jvalid && d < D) ? load16(qp + d) : u32x4{0, 0, 0, 0});
    }
  }

  f32x16 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const float c = a.scale_log2;

  const uint16_t *kbase = a.k.p + b * a.k.sb + (int64_t)h * a.k.sh;
  const uint16_t *vbase = a.v.p + b * a.v.sb + (int64_t)h * a.v.sh;

  for (int kb = ks0; kb < ks1; kb += kBN) {
    // Stage K rows [kb, kb+64) row-major; keys >= ks1 and features >= D are zero.
    for (int cidx = tid; cidx < kBN * (DP / 8); cidx += 256) {
      const int key = cidx / (DP / 8), dcc = cidx % (DP / 8);
      const int tok = kb + key;
      const u32x4 val = (tok < ks1 && dcc * 8 < D) ? load16(kbase + (int64_t)tok * a.k.st + dcc * 8)
                                                   : u32x4{0, 0, 0, 0};
      store16(&Ks[key * KP + dcc * 8], val);
    }
    // Stage V transposed: a lane takes keys (2kp, 2kp+1) at one 8-feature chunk
    // and writes 8 packed key pairs.
    for (int cidx = tid; cidx < (kBN / 2) * (DP / 8); cidx += 256) {
      const int kp = cidx % (kBN / 2), dcc = cidx / (kBN / 2);
      const int tok = kb + 2 * kp;
      const bool dok = dcc * 8 < D;
      const u32x4 v0 = (tok < ks1 && dok) ? load16(vbase + (int64_t)tok * a.v.st + dcc * 8) : u32x4{0, 0, 0, 0};
      const u32x4 v1 = (tok + 1 < ks1 && dok) ? load16(vbase + (int64_t)(tok + 1) * a.v.st + dcc * 8)
                                              : u32x4{0, 0, 0, 0};
      uint32_t *dst = reinterpret_cast<uint32_t *>(&Vt[(dcc * 8) * VP + 2 * kp]);
      constexpr int row32 = VP / 2;
      dst[0 * row32] = (v0.x & 0xffffu) | (v1.x << 16);
      dst[1 * row32] = (v0.x >> 16) | (v1.x & 0xffff0000u);
      dst[2 * row32] = (v0.y & 0xffffu) | (v1.y << 16);
      dst[3 * row32] = (v0.y >> 16) | (v1.y & 0xffff0000u);
      dst[4 * row32] = (v0.z & 0xffffu) | (v1.z << 16);
      dst[5 * row32] = (v0.z >> 16) | (v1.z & 0xffff0000u);
      dst[6 * row32] = (v0.w & 0xffffu) | (v1.w << 16);
      dst[7 * row32] = (v0.w >> 16) | (v1.w & 0xffff0000u);
    }
    __syncthreads();

    if (wave_active && kb <= wave_kmax) {
      // S^T for keys kb + [0,32) and kb + [32,64).
      f32x16 s[2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kt][r] = 0.0f;
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) {
          const bf16x8 ka = as_bf16x8(*reinterpret_cast<const u32x4 *>(&Ks[(kt * 32 + col) * KP + ds * 16 + half * 8]));
          s[kt] = mfma32(ka, qf[ds], s[kt]);
        }
      }
      // Mask keys past this column's causal limit or past the split.
      const bool need_mask = (kb + kBN - 1 > wave_kmin) || (kb + kBN > ks1);
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if (need_mask) {
            const int key = kb + kt * 32 + 8 * (r / 4) + 4 * half + (r % 4);
            if (key > lim || key >= ks1) s[kt][r] = -INFINITY;
          }
          mx = fmaxf(mx, s[kt][r]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx * c);
      const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      float psum = 0.0f;
      bf16x8 pb[2][2];
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          u32x4 w;
          float pv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) pv[e] = fast_exp2(fmaf(s[kt][hh * 8 + e], c, -m_use));
          w.x = pack_bf16x2(pv[0], pv[1]);
          w.y = pack_bf16x2(pv[2], pv[3]);
          w.z = pack_bf16x2(pv[4], pv[5]);
          w.w = pack_bf16x2(pv[6], pv[7]);
          // The normaliser sums the bf16 weights the PV product actually uses,
          // so the output stays an exact convex combination of the values.
          psum += (bf16_lo(w.x) + bf16_hi(w.x)) + (bf16_lo(w.y) + bf16_hi(w.y)) +
                  (bf16_lo(w.z) + bf16_hi(w.z)) + (bf16_lo(w.w) + bf16_hi(w.w));
          pb[kt][hh] = as_bf16x8(w);
        }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] *= alpha;
      // O^T += V^T P^T.  Lane half `half` supplies k-slots holding keys
      // kb + 32kt + 16hh + 4half + {0..3} and + 8 + {0..3} (the S^T C rows it owns).
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const uint16_t *vp = &Vt[(t * 32 + col) * VP + kt * 32 + hh * 16 + half * 4];
            const u32x2 lo = *reinterpret_cast<const u32x2 *>(vp);
            const u32x2 hi = *reinterpret_cast<const u32x2 *>(vp + 8);
            const bf16x8 va = as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y});
            acc[t] = mfma32(va, pb[kt][hh], acc[t]);
          }
    }
    __syncthreads();
  }

  // Epilogue.  acc[t][r] = O^T[d = 32t + 8(r/4) + 4half + r%4][column j].
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (!jvalid) return;
  if (rs.nsplit == 1) {
    const float inv = 1.0f / l_tot;
    uint16_t *dst = a.out + b * a.o_sb + (int64_t)(h * G + g) * a.o_sh + (int64_t)qi * a.o_st;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = t * 32 + 8 * r4 + 4 * half;
        if (d < D) {
          u32x2 w;
          w.x = pack_bf16x2(acc[t][r4 * 4 + 0] * inv, acc[t][r4 * 4 + 1] * inv);
          w.y = pack_bf16x2(acc[t][r4 * 4 + 2] * inv, acc[t][r4 * 4 + 3] * inv);
          *reinterpret_cast<u32x2 *>(dst + d) = w;
        }
      }
  } else {
    const int64_t rec = rs.rec_begin + ((int64_t)h * rs.nsplit + split) * qrows + j;
    float *po = a.part_o + rec * D;
#pragma unroll
    for (int t = 0; t < NDT; ++t)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = t * 32 + 8 * r4 + 4 * half;
        if (d < D)
          *reinterpret_cast<f32x4 *>(po + d) =
              f32x4{acc[t][r4 * 4 + 0], acc[t][r4 * 4 + 1], acc[t][r4 * 4 + 2], acc[t][r4 * 4 + 3]};
      }
    if (half == 0) {
      a.part_ml[2 * rec] = m_run;
      a.part_ml[2 * rec + 1] = l_tot;
    }
  }
}

hipError_t launch_prefill(const AttnArgs &a, int dp, int items, hipStream_t stream) {
  switch (dp) {
    case 64: hipLaunchKernelGGL(prefill_kernel<64>, dim3(items), dim3(256), 0, stream, a); break;
    case 128: hipLaunchKernelGGL(prefill_kernel<128>, dim3(items), dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL(prefill_kernel<256>, dim3(items), dim3(256), 0, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace xattn
