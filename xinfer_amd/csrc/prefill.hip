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
// Waves: four query groups of 32 vectors x KH key halves.  With KH = 2 (head
// dim 128) a block is 8 waves, two per SIMD, so one wave's MFMAs overlap the
// other's softmax; wave w+4 takes keys 32..63 of every 64-key tile and is
// merged into wave w at the end.  Each wave computes the transposed problem
// with v_mfma_f32_32x32x16_bf16:
//   S^T[key, j]  = K[key, :] . Q[j, :]      A = K tile (LDS), B = Q^T (registers)
//   O^T[d, j]   += V^T[d, key] P^T[key, j]  A = V^T tile (LDS), B = P^T (from S^T)
// so a lane's accumulator column is one query vector: the online-softmax max /
// sum are per lane (plus one exchange with lane^32) and the S^T accumulator
// registers are directly the PV B operand.  K is staged row-major, V transposed
// ([d][key]); the next tile's global loads are issued into registers before the
// current tile is computed and stored to LDS after it.
//
// MFMA 32x32x16 lane layout used (A: 32xK16, B: K16x32, C: 32x32):
//   A lane l: row l%32, k = 8*(l/32) + 0..7      B lane l: col l%32, same k
//   C lane l, reg r: row 8*(r/4) + 4*(l/32) + r%4, col l%32
// The PV product contracts over keys; the key <-> k-slot assignment only has to
// agree between the A and B operands, and both are derived from the C layout.
//
// Several splits of a tile write fp32 partial records, combined by merge.hip.
// The tile-0 / split-0 item zeroes the row's padded queries (t >= count).
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

template <int DP, int KH>
struct PrefillShape {
  static constexpr int THREADS = 256 * KH;
  static constexpr int KP = DP + 8;   // K tile pitch (bf16); 16-byte pad against bank conflicts
  static constexpr int VP = kBN + 8;  // V^T tile pitch
  static constexpr int NDS = DP / 16; // k-steps of the QK product
  static constexpr int NDT = DP / 32; // 32-row d tiles of the output
  static constexpr int KCH = kBN * (DP / 8) / THREADS;        // K 16-byte chunks per thread
  static constexpr int VCH = (kBN / 2) * (DP / 8) / THREADS;  // V key-pair chunks per thread
};

template <int DP, int KH>
__global__ void __launch_bounds__(256 * KH) prefill_kernel(const AttnArgs a) {
  using S = PrefillShape<DP, KH>;
  constexpr int THREADS = S::THREADS, KP = S::KP, VP = S::VP, NDS = S::NDS, NDT = S::NDT;
  constexpr int KCH = S::KCH, VCH = S::VCH;
  constexpr int KEYS_PER_WAVE = kBN / KH;  // keys of each tile this wave owns
  constexpr int NKT = KEYS_PER_WAVE / 32;  // 32-key sub-tiles per wave per tile
  static_assert(KCH >= 1 && VCH >= 1, "tile staging needs at least one chunk per thread");
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kBN * KP];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[DP * VP];
  __shared__ float xchg[KH > 1 ? 4 : 1][KH > 1 ? NDT * 16 + 2 : 1][64];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;
  const int qgroup = wave & 3, khalf = wave >> 2;

  const int item = blockIdx.x;
  const RowSched rs = a.rows[find_row(a.rows, a.nrows, item)];
  const int local = item - rs.item_begin;
  const int per_head = rs.ntiles * rs.nsplit;
  const int h = local / per_head;
  const int tile = (local - h * per_head) / rs.nsplit;
  const int split = local - h * per_head - tile * rs.nsplit;
  const int b = rs.batch, L = rs.length, cnt = rs.count, G = a.G, D = a.D;
  const int qrows = cnt * G, p0 = L - cnt;

  if (tile == 0 && split == 0 && cnt < a.T) {  // zero the row's padded queries
    const int per = (a.T - cnt) * D / 8;
    for (int idx = tid; idx < G * per; idx += THREADS) {
      const int g = idx / per, rest = idx - g * per;
      store16(a.out + b * a.o_sb + (int64_t)(h * G + g) * a.o_sh + (int64_t)cnt * a.o_st + rest * 8,
              u32x4{0, 0, 0, 0});
    }
  }

  // Key range of this tile and split.
  const int j_last = min(tile * kTileQ + kTileQ, qrows) - 1;
  const int kend = p0 + j_last / G + 1;
  int ks0, ks1;
  split_range(kend, rs.nsplit, split, ks0, ks1);

  // This lane's query vector.
  const int j = tile * kTileQ + qgroup * 32 + col;
  const bool jvalid = j < qrows;
  const int g = j % G, qi = j / G;
  const int lim = p0 + qi;  // last visible key
  const int jw_first = tile * kTileQ + qgroup * 32;
  const bool wave_active = jw_first < qrows;
  const int wave_kmax = p0 + (min(jw_first + 31, qrows - 1)) / G;  // last key any column sees
  const int wave_kmin = p0 + jw_first / G;                          // last key of the first column

  // Loads are unconditional, from addresses clamped into the valid range (last
  // query vector, last key of the split, last feature chunk), so they issue
  // without branches.  Clamped query features are zeroed; clamped keys are
  // masked on the scores; clamped features past D only meet zero query
  // features or land in output rows >= D, which are never stored.
  bf16x8 qf[NDS];
  {
    const int jc = jvalid ? j : qrows - 1;
    const uint16_t *qp = a.q.p + b * a.q.sb + (int64_t)(h * G + jc % G) * a.q.sh + (int64_t)(jc / G) * a.q.st;
    u32x4 raw[NDS];
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) raw[ds] = load16(qp + min(ds * 16 + half * 8, D - 8));
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
      qf[ds] = as_bf16x8((jvalid && ds * 16 + half * 8 < D) ? raw[ds] : u32x4{0, 0, 0, 0});
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

  // Register staging of one tile: K chunks (key, 8 features) and V key pairs.
  u32x4 kst[KCH], vst0[VCH], vst1[VCH];
  auto load_tile = [&](int kb) {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int cidx = tid + i * THREADS;
      const int key = cidx / (DP / 8), dcc = min(cidx % (DP / 8), D / 8 - 1);
      const int tok = min(kb + key, ks1 - 1);
      kst[i] = load16(kbase + (int64_t)tok * a.k.st + dcc * 8);
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int cidx = tid + i * THREADS;
      const int kp = cidx % (kBN / 2), dcc = min(cidx / (kBN / 2), D / 8 - 1);
      const int tok0 = min(kb + 2 * kp, ks1 - 1), tok1 = min(kb + 2 * kp + 1, ks1 - 1);
      vst0[i] = load16(vbase + (int64_t)tok0 * a.v.st + dcc * 8);
      vst1[i] = load16(vbase + (int64_t)tok1 * a.v.st + dcc * 8);
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < KCH; ++i) {
      const int cidx = tid + i * THREADS;
      const int key = cidx / (DP / 8), dcc = cidx % (DP / 8);
      store16(&Ks[key * KP + dcc * 8], kst[i]);
    }
#pragma unroll
    for (int i = 0; i < VCH; ++i) {
      const int cidx = tid + i * THREADS;
      const int kp = cidx % (kBN / 2), dcc = cidx / (kBN / 2);
      const u32x4 v0 = vst0[i], v1 = vst1[i];
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
  };

  if (ks0 < ks1) {
    load_tile(ks0);
    store_tile();
  }
  __syncthreads();
  for (int kb = ks0; kb < ks1; kb += kBN) {
    const bool has_next = kb + kBN < ks1;
    if (has_next) load_tile(kb + kBN);  // in flight while this tile is computed

    const int kw = kb + khalf * KEYS_PER_WAVE;  // first key of this wave's share
    if (wave_active && kw <= wave_kmax && kw < ks1) {
      f32x16 s[NKT];
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kt][r] = 0.0f;
#pragma unroll
        for (int ds = 0; ds < NDS; ++ds) {
          const bf16x8 ka = as_bf16x8(*reinterpret_cast<const u32x4 *>(
              &Ks[(khalf * KEYS_PER_WAVE + kt * 32 + col) * KP + ds * 16 + half * 8]));
          s[kt] = mfma32(ka, qf[ds], s[kt]);
        }
      }
      // Mask keys past this column's causal limit or past the split.
      const bool need_mask = (kw + KEYS_PER_WAVE - 1 > wave_kmin) || (kw + KEYS_PER_WAVE > ks1);
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if (need_mask) {
            const int key = kw + kt * 32 + 8 * (r / 4) + 4 * half + (r % 4);
            if (key > lim || key >= ks1) s[kt][r] = -INFINITY;
          }
          mx = fmaxf(mx, s[kt][r]);
        }
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx * c);
      const float m_use = (m_new == -INFINITY) ? 0.0f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      float psum = 0.0f;
      bf16x8 pb[NKT][2];
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          float pv[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) pv[e] = fast_exp2(fmaf(s[kt][hh * 8 + e], c, -m_use));
          u32x4 w;
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
      // kw + 32kt + 16hh + 4half + {0..3} and + 8 + {0..3} (the S^T C rows it owns).
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const uint16_t *vp = &Vt[(t * 32 + col) * VP + khalf * KEYS_PER_WAVE + kt * 32 + hh * 16 + half * 4];
            const u32x2 lo = *reinterpret_cast<const u32x2 *>(vp);
            const u32x2 hi = *reinterpret_cast<const u32x2 *>(vp + 8);
            acc[t] = mfma32(as_bf16x8(u32x4{lo.x, lo.y, hi.x, hi.y}), pb[kt][hh], acc[t]);
          }
    }
    __syncthreads();  // every wave is done with this tile
    if (has_next) {
      store_tile();
      __syncthreads();
    }
  }

  // Per-lane partial sum -> column sum (lanes l and l^32 hold the two key halves of a 32x32 tile).
  l_run += __shfl_xor(l_run, 32);
  if constexpr (KH > 1) {
    // Fold the second key half (waves 4..7) into waves 0..3.
    if (khalf == 1) {
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) xchg[qgroup][t * 16 + r][lane] = acc[t][r];
      xchg[qgroup][NDT * 16][lane] = m_run;
      xchg[qgroup][NDT * 16 + 1][lane] = l_run;
    }
    __syncthreads();
    if (khalf == 0) {
      const float m_b = xchg[qgroup][NDT * 16][lane], l_b = xchg[qgroup][NDT * 16 + 1][lane];
      const float mx = fmaxf(m_run, m_b);
      const float mu = mx == -INFINITY ? 0.0f : mx;
      const float wa = fast_exp2(m_run - mu), wb = fast_exp2(m_b - mu);
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = acc[t][r] * wa + xchg[qgroup][t * 16 + r][lane] * wb;
      l_run = l_run * wa + l_b * wb;
      m_run = mx;
    }
  }

  // Epilogue (waves 0..3).  acc[t][r] = O^T[d = 32t + 8(r/4) + 4half + r%4][column j].
  if (khalf == 0 && jvalid) {
    if (rs.nsplit == 1) {
      const float inv = 1.0f / l_run;
      uint16_t *dst = a.out + b * a.o_sb + (int64_t)(h * G + g) * a.o_sh + (int64_t)qi * a.o_st;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int d = t * 32 + 8 * r4 + 4 * half;
          if (d < D)
            *reinterpret_cast<u32x2 *>(dst + d) =
                u32x2{pack_bf16x2(acc[t][r4 * 4 + 0] * inv, acc[t][r4 * 4 + 1] * inv),
                      pack_bf16x2(acc[t][r4 * 4 + 2] * inv, acc[t][r4 * 4 + 3] * inv)};
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
        a.part_ml[2 * rec + 1] = l_run;
      }
    }
  }
}

hipError_t launch_prefill(const AttnArgs &a, int dp, int items, hipStream_t stream) {
  switch (dp) {
    case 64: hipLaunchKernelGGL((prefill_kernel<64, 1>), dim3(items), dim3(256), 0, stream, a); break;
    case 128: hipLaunchKernelGGL((prefill_kernel<128, 2>), dim3(items), dim3(512), 0, stream, a); break;
    default: hipLaunchKernelGGL((prefill_kernel<256, 1>), dim3(items), dim3(256), 0, stream, a); break;
  }
  return hipGetLastError();
}

}  // namespace xattn
