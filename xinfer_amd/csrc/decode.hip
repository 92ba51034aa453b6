// Split-KV decode attention for rows with few query vectors per KV head
// (G * count <= 8): the q_len = 1 decode step and short appended chunks.
//
// Replaces, for those rows, the ATen FlashAttention-2 call of
// compiler/common/kernels/attention.cpp:66-72 / :116-117.  Math: for every
// query vector j = i*G + g of KV head h in row r,
//   out_j = sum_t softmax_t(scale * q_j . k_t) v_t  over keys t <= L - count + i
// (lower-right causal), fp32 scores / softmax / accumulation, bf16 in and out.
//
// Work item = (row, kv head, chunk of TOK_ITEM keys); the chunk's K and V are
// read from HBM exactly once and shared by the G grouped query heads.  One
// block per item; every K/V load of the block (8 rows of 16 bytes per lane and
// tensor, 4 for 8 query vectors) is issued before any arithmetic, and the small
// register footprint keeps several blocks resident per CU, so the loads of
// some blocks are in flight while others compute (measured on MI355X: 32 KB
// per tensor per block is the read shape that sustains the most bandwidth).
//
// A block is 4 waves, each owning a contiguous quarter of the item.  LPT lanes
// hold one key row, CPL 16-byte chunks each (chunks dc, dc + LPT, ...), so a
// wave instruction reads one 16-byte chunk of each lane, TPW = 64/LPT rows
// (1 KB in runs of LPT*16 bytes).  K and V are read with raw
// buffer loads: the (row, head) base in scalar registers, a 32-bit lane offset
// and a scalar per-row offset, so a load costs no vector address arithmetic;
// the resource ends at the item's last key, and loads past it return zero
// without touching memory.  Per key row: bf16 dot2 against the lane's 8 query
// features and a DPP all-reduce over the LPT lanes of the row; then one max
// over the wave's rows (all of them are in registers, so no online rescale),
// and the fp32 weights and accumulation, all lane-local.  The four waves are
// combined through LDS.
//
// One chunk per (row, head): the block writes normalised bf16 output.  Several
// chunks: each writes an fp32 partial record per query vector, combined by
// merge.hip.  The schedule depends only on the lengths, so results are
// deterministic and a row's output never depends on another row's data.
//
// K and V are streamed with non-temporal loads (each byte is read once):
// measured on MI355X, 10% faster than default-policy loads.
// Padded queries (t >= count) get zeros from the row's first item; a row with
// count == 0 is scheduled only for that.
#include "device_common.h"
#include "kernel_args.h"
#include "launch.h"

namespace xattn {

template <int DP, int QR>
struct DecodeShape {
  // 16-byte chunks of a key row per lane.  Measured on MI355X: two chunks
  // per lane for D = 256 (16 lanes per row, half the reduction steps per
  // byte) lowers the occupancy of the four-query-vector kernel from 4 to 3
  // waves per SIMD and is 2 us slower on a 122 MB decode batch.
  static constexpr int CPL = 1;
  static constexpr int LPT = DP / (8 * CPL);     // lanes per key row
  static constexpr int TPW = 64 / LPT;           // key rows per wave instruction
  // Key rows per lane per item: 16 KB of K+V per wave (8 KB for 8 query
  // vectors, whose accumulators take the registers).
  static constexpr int ROWS = (QR == 8 ? 8 : 16) / (2 * CPL);
  static constexpr int U0 = QR <= 2 ? 4 : (QR == 4 ? 2 : 1);
  static constexpr int U = U0 < ROWS ? U0 : ROWS;  // rows per lane per block
  static constexpr int NB = ROWS / U;            // blocks per wave per item
  static constexpr int BLK = TPW * U;            // keys per wave block
  static constexpr int TOK_WAVE = NB * BLK;      // keys per wave per round
  static constexpr int TOK_ROUND = 4 * TOK_WAVE; // keys per block per round
};

// An item takes ROUNDS rounds: the block loads and computes TOK_ROUND keys at
// a time, reusing the registers, and writes one output or record per item.
// The planner takes four rounds for launches that have many items and one
// otherwise.  Measured on MI355X (decode + merge kernels): a 122 MB D = 256
// batch 35.3 us with one round, 32.8 with two, 34.1 with three, 31.2 with
// four, 31.7 with eight; a 126 MB D = 128 batch 27.7, 27.9, 28.4, 27.3 and
// 34.9 (with eight, fewer blocks than CUs); batches of 45-98 MB were neutral
// to 0.6 us slower with two rounds, and small batches slower, with too few
// blocks.
constexpr int kDecodeRounds = kDecodeItemRounds;

struct DecodeItem {
  int b, h, split, nsplit, cnt, L, t0, t1;
  int kvb;    // cache row of the item's K/V: b, or b's page
  int first;  // item of split 0 of this (row, kv head)
  int64_t rec_begin;
};

// The arguments a decode block uses (named as in AttnArgs), pinned in SGPRs by
// the kernel's prologue.
struct DecodeParams {
  View q, k, v;
  uint16_t *out;
  int64_t o_sb, o_sh, o_st;
  float *part_o, *part_ml;
  float scale_log2;
  int32_t D, G, T;
  uint64_t *arrive_ctr;  // in-launch merge (merge_in_launch), else null
  uint64_t tag;
};

__device__ __forceinline__ DecodeItem locate_item(const RowSched &rs, int item, int tok_item) {
  DecodeItem it;
  const int local = item - rs.item_begin;
  it.h = local / rs.nsplit;
  it.split = local - it.h * rs.nsplit;
  it.nsplit = rs.nsplit;
  it.b = rs.batch;
  it.kvb = rs.batch;
  it.cnt = rs.count;
  it.L = rs.length;
  it.t0 = it.split * tok_item;
  it.t1 = min(it.L, it.t0 + tok_item);
  it.first = rs.item_begin + it.h * rs.nsplit;
  it.rec_begin = rs.rec_begin;
  return it;
}

// Registers of one in-flight item: its K/V rows and query features.
template <int DP, int QR>
struct DecodeRegs {
  using S = DecodeShape<DP, QR>;
  u32x4 k[S::NB][S::U][S::CPL], v[S::NB][S::U][S::CPL], q[QR][S::CPL];
};

// The c-th chunk of a key row this lane holds, clamped into the row (lanes
// past D re-read the row's last chunk: bytes of the row itself, never the gap
// after it, which a padded view may fill with anything).
template <int DP, int QR>
__device__ __forceinline__ int lane_chunk(int dc, int c, int D) {
  const int chunk = dc + c * DecodeShape<DP, QR>::LPT;
  return chunk * 8 < D ? chunk : D / 8 - 1;
}

// Zero out[b, h*G + g, t, :] for g < G and t in [t_begin, T).
__device__ __forceinline__ void zero_queries(const DecodeParams &a, int b, int h, int t_begin) {
  const int chunks = a.D / 8;                       // 16-byte chunks per query row
  const int per_head = (a.T - t_begin) * chunks;
  for (int idx = threadIdx.x; idx < a.G * per_head; idx += blockDim.x) {
    const int g = idx / per_head, rest = idx - g * per_head;
    const int t = t_begin + rest / chunks, c = rest - (rest / chunks) * chunks;
    store16(a.out + b * a.o_sb + (int64_t)(h * a.G + g) * a.o_sh + (int64_t)t * a.o_st + c * 8,
            u32x4{0, 0, 0, 0});
  }
}

// Query features of the item's vectors (clamped into the row; zeroed past D later).
template <int DP, int QR>
__device__ __forceinline__ void load_query(const DecodeParams &a, const DecodeItem &it, DecodeRegs<DP, QR> &r, int dc) {
  const int qrows = it.cnt * a.G;
#pragma unroll
  for (int j = 0; j < QR; ++j) {
    const int jc = j < qrows ? j : qrows - 1;
    const uint16_t *qrow = a.q.p + it.b * a.q.sb + (int64_t)(it.h * a.G + jc % a.G) * a.q.sh + (int64_t)(jc / a.G) * a.q.st;
#pragma unroll
    for (int c = 0; c < DecodeShape<DP, QR>::CPL; ++c) r.q[j][c] = load16(qrow + lane_chunk<DP, QR>(dc, c, a.D) * 8);
  }
}

// Issue every load of one round of an item: K/V rows through buffer resources
// ending at the item's last key, and (round 0) the query features (clamped
// into the row, zeroed past D).
template <int DP, int QR>
__device__ __forceinline__ void issue_item(const DecodeParams &a, const DecodeItem &it, DecodeRegs<DP, QR> &r,
                                           int wave, int slot, int dc, int round = 0, int part = 0) {
  using S = DecodeShape<DP, QR>;
  if (it.cnt == 0) return;
  // The query first: its loads complete before the K/V rows the first dot needs.
  if constexpr (QR <= 4) {
    if (round == 0 && part == 0) load_query(a, it, r, dc);  // wider groups load it in process_item
  }
  const uint32_t row_bytes_k = (uint32_t)(a.k.st * 2), row_bytes_v = (uint32_t)(a.v.st * 2);
  const auto rk = buffer_rsrc(a.k.p + it.kvb * a.k.sb + (int64_t)it.h * a.k.sh, (uint32_t)it.t1 * row_bytes_k);
  const auto rv = buffer_rsrc(a.v.p + it.kvb * a.v.sb + (int64_t)it.h * a.v.sh, (uint32_t)it.t1 * row_bytes_v);
  const int first = it.t0 + round * S::TOK_ROUND + wave * S::TOK_WAVE + slot;  // this lane's first key row
  // Chunks past D (padded head dims) are clamped into the row; their query
  // features are zero and their sums are not written.
  uint32_t vk[S::CPL], vv[S::CPL];
#pragma unroll
  for (int c = 0; c < S::CPL; ++c) {
    const uint32_t chunk = (uint32_t)lane_chunk<DP, QR>(dc, c, a.D);
    vk[c] = (uint32_t)first * row_bytes_k + chunk * 16;
    vv[c] = (uint32_t)first * row_bytes_v + chunk * 16;
  }
  // Every K row before any V row: the scores need all of K, the weights none of V.
  if (part != 2)
#pragma unroll
  for (int nb = 0; nb < S::NB; ++nb)
#pragma unroll
    for (int u = 0; u < S::U; ++u)
#pragma unroll
      for (int c = 0; c < S::CPL; ++c)
        r.k[nb][u][c] = buffer_load16_stream(rk, vk[c], (nb * S::BLK + u * S::TPW) * row_bytes_k);
  if (part != 1)
#pragma unroll
  for (int nb = 0; nb < S::NB; ++nb)
#pragma unroll
    for (int u = 0; u < S::U; ++u)
#pragma unroll
      for (int c = 0; c < S::CPL; ++c)
        r.v[nb][u][c] = buffer_load16_stream(rv, vv[c], (nb * S::BLK + u * S::TPW) * row_bytes_v);
}

template <int DP, int QR>
struct DecodeShared {
  float red_o[4][QR][DP];
  float red_m[4][QR], red_l[4][QR];
};

// In-launch merge of one (row, kv head)'s split records, called by every
// thread of a block that has just written its records (AttnArgs::arrive_ctr
// set).  The planner takes this path only for launches whose split rows have
// at most kMergeSerialSplits splits and whose Hkv is a multiple of 8, and the
// kernel then runs every split of a (row, kv head) on one XCD (block b on XCD
// b % 8, which probe_xcd_dispatch checks once per device), so the records meet
// in that XCD's L2.  Each block, once its record stores are acknowledged,
// counts its arrival on the (row, kv head)'s counter; the last to arrive reads
// the records past its CU's L1 and folds them as merge.hip's one-thread-per-
// (vector, 4 features) layout does -- splits in increasing order, with the
// products fused as that kernel compiles them (l = fma(l_old, a, ls w), o =
// fma(os, w, o_old a)) -- so that both paths give the same bits, and resets
// the counter to zero.
//
// Counter word: arrivals (bits 0-11), XCC of the first arrival (12-15),
// arrivals from another XCC (16-27), the launch's tag (28-63).  The first
// arrival claims a word that does not carry this launch's tag (zero after the
// previous launch's reset, or whatever the workspace held) by compare-and-
// swap; every other arrival adds itself with one fetch-and-add, so no arrival
// waits behind another.  A (row, kv head) whose splits ran on more than one
// XCC gets NaN outputs rather than a fold of records another L2 may hold.
template <int DP>
__device__ void merge_in_launch(const DecodeParams &a, const DecodeItem &it, int qrows) {
  __shared__ uint32_t arrival;
  const int tid = threadIdx.x;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's record stores are acknowledged
  __syncthreads();
  if (tid == 0) {
    uint32_t xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 15u;
    uint64_t *const ctr = a.arrive_ctr + it.first;
    const uint64_t tag = a.tag;
    uint64_t seen = 0;
    bool claimed = false;
    // Ends after at most two attempts: only this launch's first arrival
    // writes its tag, and no reset happens before every arrival is counted.
    while ((seen >> 28) != tag) {
      if (__hip_atomic_compare_exchange_strong(ctr, &seen, (tag << 28) | ((uint64_t)xcc << 12) | 1u,
                                               __ATOMIC_RELAXED, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) {
        claimed = true;
        break;
      }
    }
    uint32_t count = 1, mixed = 0;
    if (!claimed) {
      const bool other = ((seen >> 12) & 15u) != xcc;
      const uint64_t before = __hip_atomic_fetch_add(ctr, (uint64_t)1 + (other ? (uint64_t)1 << 16 : 0),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      count = (uint32_t)(before & 0xfffu) + 1;
      mixed = (uint32_t)((before >> 16) & 0xfffu) + (other ? 1u : 0u);
    }
    const bool last = count == (uint32_t)it.nsplit;
    if (last) __hip_atomic_store(ctr, (uint64_t)0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    arrival = !last ? 0u : (mixed == 0 ? 1u : 2u);
  }
  __syncthreads();
  const uint32_t flag = arrival;
  if (flag == 0) return;

  constexpr int FQ = DP / 4;  // feature quads of a padded vector
  const int D = a.D, G = a.G, nsplit = it.nsplit;
  // Record (split s, vector j) of this (row, kv head): rec0 + s * qrows + j.
  const int64_t rec0 = it.rec_begin + (int64_t)it.h * nsplit * qrows;
  const __amdgpu_buffer_rsrc_t o_rsrc = buffer_rsrc(a.part_o + rec0 * D, (uint32_t)(nsplit * qrows * D * 4));
  const __amdgpu_buffer_rsrc_t ml_rsrc = buffer_rsrc(a.part_ml + 2 * rec0, (uint32_t)(nsplit * qrows * 8));
  for (int idx = tid; idx < qrows * FQ; idx += blockDim.x) {
    const int j = idx / FQ, f = idx - j * FQ;
    if (f * 4 >= D) continue;
    u32x2 ml[kMergeSerialSplits];
    u32x4 o[kMergeSerialSplits];
#pragma unroll
    for (int s = 0; s < kMergeSerialSplits; ++s)
      if (s < nsplit) {
        ml[s] = buffer_load8_l2(ml_rsrc, (uint32_t)((s * qrows + j) * 8));
        o[s] = buffer_load16_l2(o_rsrc, (uint32_t)(((s * qrows + j) * D + 4 * f) * 4));
      }
    float m = -INFINITY, l = 0.0f;
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < kMergeSerialSplits; ++s) {
      if (s >= nsplit) break;
      const float ms = __uint_as_float(ml[s].x);
      if (ms == -INFINITY) continue;
      const float ls = __uint_as_float(ml[s].y);
      const f32x4 os = __builtin_bit_cast(f32x4, o[s]);
      const float mn = fmaxf(m, ms);
      const float wa = fast_exp2(m - mn), ws = fast_exp2(ms - mn);  // m = -inf -> wa = 0
      l = __builtin_fmaf(l, wa, ls * ws);
      acc = f32x4{__builtin_fmaf(os.x, ws, acc.x * wa), __builtin_fmaf(os.y, ws, acc.y * wa),
                  __builtin_fmaf(os.z, ws, acc.z * wa), __builtin_fmaf(os.w, ws, acc.w * wa)};
      m = mn;
    }
    const float inv = 1.0f / l;
    uint16_t *dst = a.out + it.b * a.o_sb + (int64_t)(it.h * G + j % G) * a.o_sh + (int64_t)(j / G) * a.o_st + 4 * f;
    *as_global(reinterpret_cast<u32x2 *>(dst)) =
        flag == 1 ? u32x2{pack_bf16x2(acc.x * inv, acc.y * inv), pack_bf16x2(acc.z * inv, acc.w * inv)}
                  : u32x2{0x7fc07fc0u, 0x7fc07fc0u};
  }
}

// Compute one item from its registers (round 0 already issued); writes output
// or partial records.
template <int DP, int QR, int ROUNDS>
__device__ __forceinline__ void process_item(const DecodeParams &a, const DecodeItem &it, DecodeRegs<DP, QR> &r,
                                             DecodeShared<DP, QR> &sh, int wave, int lane, int slot, int dc) {
  using S = DecodeShape<DP, QR>;
  constexpr int LPT = S::LPT, TPW = S::TPW, U = S::U, NB = S::NB, BLK = S::BLK, CPL = S::CPL;
  constexpr int F = 8 * CPL;  // output features per lane
  const int tid = threadIdx.x, G = a.G;
  if (it.cnt == 0) {
    zero_queries(a, it.b, it.h, 0);
    return;
  }
  if (it.split == 0 && it.cnt < a.T) zero_queries(a, it.b, it.h, it.cnt);
  if constexpr (QR > 4) load_query(a, it, r, dc);
  const int qrows = it.cnt * G;
  const float c = a.scale_log2;
  int lim[QR];
#pragma unroll
  for (int j = 0; j < QR; ++j) {
    lim[j] = j < qrows ? it.L - it.cnt + j / G : -1;  // last visible key of query vector j
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc)
      if (!(j < qrows && (dc + cc * LPT) * 8 < a.D)) r.q[j][cc] = u32x4{0, 0, 0, 0};
  }

  // A round's keys are all in registers, so within a round the softmax needs
  // no online rescale: every score first (masked to -inf), then the max over
  // the wave's keys of the round (log2 units, the same on every lane), then
  // the weights and the accumulation against the running max m, which the
  // round's max may raise once (one rescale of the accumulators per round).
  float sc[NB][QR][U], m[QR], l[QR], acc[QR][F];
  auto score = [&](int nb, int j, int u) {
    float d = 0.0f;
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc) d = dot8_bf16(r.k[nb][u][cc], r.q[j][cc], d);
    return group_sum<LPT>(d);
  };
  // Two or four query vectors over 16 or 32 lanes per key row: reduce-scatter
  // the dot products, so each lane takes the score, weight and row sum of one
  // query (lane & (QR - 1)) instead of all of them, and fetches the other
  // queries' weights from its quad for the accumulation.
  constexpr bool RS = (QR == 2 || QR == 4) && (LPT == 16 || LPT == 32) && CPL == 1;
  if constexpr (RS) {
    const int jq = lane & (QR - 1);
    int lim_q = lim[0];
#pragma unroll
    for (int j = 1; j < QR; ++j) lim_q = jq == j ? lim[j] : lim_q;
    float scq[NB][U], lq = 0.0f;
    auto score_q = [&](int nb, int u) {
      float d[QR];
#pragma unroll
      for (int j = 0; j < QR; ++j) d[j] = dot8_bf16(r.k[nb][u][0], r.q[j][0], 0.0f);
      return rs_sum<QR, LPT>(d, lane);
    };
#pragma unroll
    for (int round = 0; round < ROUNDS; ++round) {
      if (round > 0 && it.t0 + round * S::TOK_ROUND >= it.t1) break;  // block-uniform: the item ends earlier
      // The next round's rows are loaded while this one computes: K once the
      // scores have read this round's K, V once the accumulation has read V.
      const bool next = round + 1 < ROUNDS && it.t0 + (round + 1) * S::TOK_ROUND < it.t1;
      const int wb = it.t0 + round * S::TOK_ROUND + wave * S::TOK_WAVE;
      const int we = min(it.t1, wb + S::TOK_WAVE);
      const bool masked = wb + S::TOK_WAVE > we || wb + S::TOK_WAVE - 1 > it.L - it.cnt;
      if (masked) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int tok = wb + nb * BLK + u * TPW + slot;
            const float sv = score_q(nb, u);
            scq[nb][u] = (tok < we && tok <= lim_q) ? sv : -INFINITY;
          }
      } else {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int u = 0; u < U; ++u) scq[nb][u] = score_q(nb, u);
      }
      if (next) issue_item(a, it, r, wave, slot, dc, round + 1, 1);
      float mx = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int u = 0; u < U; ++u) mx = fmaxf(mx, scq[nb][u]);
      const float mt_q = slot_max<LPT>(mx) * c;
      float alpha_q = 1.0f;
#pragma unroll
      for (int j = 0; j < QR; ++j) {
        float mt;
        if constexpr (QR == 4) {
          mt = j == 0 ? quad_query<4, 0>(mt_q) : j == 1 ? quad_query<4, 1>(mt_q)
                                                         : j == 2 ? quad_query<4, 2>(mt_q) : quad_query<4, 3>(mt_q);
        } else {
          mt = j == 0 ? quad_query<2, 0>(mt_q) : quad_query<2, 1>(mt_q);
        }
        if (round == 0) {
          m[j] = mt;
#pragma unroll
          for (int e = 0; e < F; ++e) acc[j][e] = 0.0f;
        } else {
          const float m_new = fmaxf(m[j], mt);
          const float alpha = fast_exp2(m[j] - (m_new == -INFINITY ? 0.0f : m_new));  // m = -inf: 0
          alpha_q = jq == j ? alpha : alpha_q;
#pragma unroll
          for (int e = 0; e < F; ++e) acc[j][e] *= alpha;
          m[j] = m_new;
        }
      }
      lq *= alpha_q;
      float mq = m[0];
#pragma unroll
      for (int j = 1; j < QR; ++j) mq = jq == j ? m[j] : mq;
      const float mu_q = mq == -INFINITY ? 0.0f : mq;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        float p[QR][U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float pq = fast_exp2(fmaf(scq[nb][u], c, -mu_q));
          lq += pq;
          if constexpr (QR == 4) {
            p[0][u] = quad_query<4, 0>(pq);
            p[1][u] = quad_query<4, 1>(pq);
            p[2][u] = quad_query<4, 2>(pq);
            p[3][u] = quad_query<4, 3>(pq);
          } else {
            p[0][u] = quad_query<2, 0>(pq);
            p[1][u] = quad_query<2, 1>(pq);
          }
        }
#pragma unroll
        for (int e = 0; e < F; ++e) {
          float vf[U];
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const uint32_t w = r.v[nb][u][e / 8][(e % 8) >> 1];
            vf[u] = (e & 1) ? bf16_hi(w) : bf16_lo(w);
          }
#pragma unroll
          for (int j = 0; j < QR; ++j) {
            float t = acc[j][e];
#pragma unroll
            for (int u = 0; u < U; ++u) t = fmaf(p[j][u], vf[u], t);
            acc[j][e] = t;
          }
        }
      }
      if (next) issue_item(a, it, r, wave, slot, dc, round + 1, 2);
    }
    if constexpr (QR == 4) {
      l[0] = quad_query<4, 0>(lq);
      l[1] = quad_query<4, 1>(lq);
      l[2] = quad_query<4, 2>(lq);
      l[3] = quad_query<4, 3>(lq);
    } else {
      l[0] = quad_query<2, 0>(lq);
      l[1] = quad_query<2, 1>(lq);
    }
  } else
#pragma unroll
  for (int round = 0; round < ROUNDS; ++round) {
    if (round > 0) {
      if (it.t0 + round * S::TOK_ROUND >= it.t1) break;  // block-uniform: the item ends earlier
      issue_item(a, it, r, wave, slot, dc, round);
    }
    const int wb = it.t0 + round * S::TOK_ROUND + wave * S::TOK_WAVE;
    const int we = min(it.t1, wb + S::TOK_WAVE);
    // Keys need masking only in a wave whose rows reach past the item (the
    // row's end) or past the first query's causal limit, L - count; query
    // vectors past qrows are never written.  The test is wave-uniform.
    const bool masked = wb + S::TOK_WAVE > we || wb + S::TOK_WAVE - 1 > it.L - it.cnt;
    if (masked) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < QR; ++j)
#pragma unroll
          for (int u = 0; u < U; ++u) {
            const int tok = wb + nb * BLK + u * TPW + slot;
            const float sv = score(nb, j, u);
            sc[nb][j][u] = (tok < we && tok <= lim[j]) ? sv : -INFINITY;
          }
    } else {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < QR; ++j)
#pragma unroll
          for (int u = 0; u < U; ++u) sc[nb][j][u] = score(nb, j, u);
    }
#pragma unroll
    for (int j = 0; j < QR; ++j) {
      float mx = -INFINITY;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int u = 0; u < U; ++u) mx = fmaxf(mx, sc[nb][j][u]);
      const float mt = slot_max<LPT>(mx) * c;
      if (round == 0) {
        m[j] = mt;
        l[j] = 0.0f;
#pragma unroll
        for (int e = 0; e < F; ++e) acc[j][e] = 0.0f;
      } else {
        const float m_new = fmaxf(m[j], mt);
        const float alpha = fast_exp2(m[j] - (m_new == -INFINITY ? 0.0f : m_new));  // m = -inf: 0
        l[j] *= alpha;
#pragma unroll
        for (int e = 0; e < F; ++e) acc[j][e] *= alpha;
        m[j] = m_new;
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      float p[QR][U];
#pragma unroll
      for (int j = 0; j < QR; ++j) {
        const float mu = m[j] == -INFINITY ? 0.0f : m[j];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          p[j][u] = fast_exp2(fmaf(sc[nb][j][u], c, -mu));
          l[j] += p[j][u];
        }
      }
#pragma unroll
      for (int e = 0; e < F; ++e) {
        float vf[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const uint32_t w = r.v[nb][u][e / 8][(e % 8) >> 1];
          vf[u] = (e & 1) ? bf16_hi(w) : bf16_lo(w);
        }
#pragma unroll
        for (int j = 0; j < QR; ++j) {
          float t = acc[j][e];
#pragma unroll
          for (int u = 0; u < U; ++u) t = fmaf(p[j][u], vf[u], t);
          acc[j][e] = t;
        }
      }
    }
  }

  // Sum over the TPW row slots of the wave (the max m is already wave-uniform).
#pragma unroll
  for (int j = 0; j < QR; ++j) {
    l[j] = slot_sum<LPT>(l[j]);
#pragma unroll
    for (int e = 0; e < F; ++e) acc[j][e] = slot_sum<LPT>(acc[j][e]);
  }
  if (slot == 0) {
#pragma unroll
    for (int cc = 0; cc < CPL; ++cc)
      if ((dc + cc * LPT) * 8 < a.D) {
#pragma unroll
        for (int j = 0; j < QR; ++j)
#pragma unroll
          for (int e = 0; e < 8; ++e) sh.red_o[wave][j][(dc + cc * LPT) * 8 + e] = acc[j][cc * 8 + e];
      }
  }
  if (lane == 0) {
#pragma unroll
    for (int j = 0; j < QR; ++j) {
      sh.red_m[wave][j] = m[j];
      sh.red_l[wave][j] = l[j];
    }
  }
  __syncthreads();

  // Combine the four waves, then write the output or a partial record.
  for (int idx = tid; idx < QR * DP; idx += 256) {
    const int j = idx / DP, d = idx % DP;
    if (j >= qrows || d >= a.D) continue;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < 4; ++w) mx = fmaxf(mx, sh.red_m[w][j]);
    const float mu = mx == -INFINITY ? 0.0f : mx;
    float o = 0.0f, lsum = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float wt = fast_exp2(sh.red_m[w][j] - mu);
      o = fmaf(wt, sh.red_o[w][j][d], o);
      lsum = fmaf(wt, sh.red_l[w][j], lsum);
    }
    if (it.nsplit == 1) {
      const int g = j % G, i = j / G;
      uint16_t *dst = a.out + it.b * a.o_sb + (int64_t)(it.h * G + g) * a.o_sh + (int64_t)i * a.o_st;
      as_global(dst)[d] = (uint16_t)f32_to_bf16_bits(o / lsum);
    } else {
      const int64_t rec = it.rec_begin + ((int64_t)it.h * it.nsplit + it.split) * qrows + j;
      as_global(a.part_o)[rec * a.D + d] = o;
      if (d == 0)
        *as_global(reinterpret_cast<u32x2 *>(a.part_ml + 2 * rec)) = u32x2{__float_as_uint(mx), __float_as_uint(lsum)};
    }
  }
  if (a.arrive_ctr != nullptr && it.nsplit > 1) merge_in_launch<DP>(a, it, qrows);
}

template <int DP, int QR, int ROUNDS>
__global__ void __launch_bounds__(256) decode_kernel(const AttnArgs a) {
  using S = DecodeShape<DP, QR>;
  __shared__ DecodeShared<DP, QR> sh;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int slot = lane / S::LPT, dc = lane % S::LPT;
  // Every argument of the block, loaded in one round trip (see XATTN_PIN_VIEW).
  RowLookup<RowSched> rows;
  rows.load(a.rows);
  int nrows = a.nrows;
  DecodeParams p{a.q,          a.k,  a.v,  a.out, a.o_sb, a.o_sh,       a.o_st, a.part_o, a.part_ml,
                 a.scale_log2, a.D,  a.G,  a.T,   a.arrive_ctr, a.tag};
  const int32_t *blocks = a.blocks;
  int64_t blocks_stride = a.blocks_stride;
  int kv_rows = a.kv_rows;
  asm volatile(""
               : XATTN_PIN_BEGINS(rows), XATTN_PIN_ROWSCHED(rows.first), "+s"(nrows), XATTN_PIN_VIEW(p.q),
                 XATTN_PIN_VIEW(p.k), XATTN_PIN_VIEW(p.v), "+s"(p.out), "+s"(p.o_sb), "+s"(p.o_sh), "+s"(p.o_st),
                 "+s"(p.part_o), "+s"(p.part_ml), "+s"(p.scale_log2), "+s"(p.D), "+s"(p.G), "+s"(p.T),
                 "+s"(blocks), "+s"(blocks_stride), "+s"(kv_rows));
  DecodeItem it;
  if (p.arrive_ctr == nullptr) {
    const int item = blockIdx.x;
    it = locate_item(rows.find(a.rows, nrows, item), item, ROUNDS * S::TOK_ROUND);
  } else {
    // In-launch merge (Hkv a multiple of 8): block b runs on XCD x = b % 8 and
    // takes, row after row, the items of the kv heads h = x (mod 8), so every
    // split of a (row, kv head) runs on one XCD and each XCD gets the same
    // work.  XCD x's list holds Hkv / 8 heads of each row: row r's part of it
    // starts at item_begin / 8.
    const int x = (int)(blockIdx.x % 8), slot = (int)(blockIdx.x / 8);
    const RowSched rs = rows.find(a.rows, nrows, 8 * slot);
    const int local = slot - rs.item_begin / 8, hh = local / rs.nsplit;
    const int h = 8 * hh + x, split = local - hh * rs.nsplit;
    it = locate_item(rs, rs.item_begin + h * rs.nsplit + split, ROUNDS * S::TOK_ROUND);
  }
  // K/V rows: the page is read while the loads issued for row it.b are in
  // flight; another page (never with the identity table) drains and reissues
  // them.
  const int raw_page = read_page(blocks, blocks_stride, it.b);
  __builtin_amdgcn_sched_barrier(0);
  DecodeRegs<DP, QR> r;
  issue_item(p, it, r, wave, slot, dc);
  __builtin_amdgcn_sched_barrier(0);
  const int page = page_in_range(raw_page, kv_rows);
  if (__builtin_expect(page != it.kvb, 0)) {
    __builtin_amdgcn_s_waitcnt(0);
    it.kvb = page;
    issue_item(p, it, r, wave, slot, dc);
  }
  process_item<DP, QR, ROUNDS>(p, it, r, sh, wave, lane, slot, dc);
}

// Graph-capture decode: the launch shape depends only on the tensor shapes.
// Each block reads every row's count and length once, numbers the row's work
// items as the default schedule would (Hkv x splits, or Hkv zero-fill items
// for a row without queries), and takes items blockIdx.x, blockIdx.x +
// gridDim.x, ... of that list (ROUNDS > 1: the grid holds every item of the
// capacity layout, and a block takes item blockIdx.x only), so the valid
// items are spread evenly over the grid whatever the lengths; blocks past the
// list exit after the one read.
template <int DP, int QR, int ROUNDS>
__global__ void __launch_bounds__(256) decode_capture_kernel(const CaptureArgs c) {
  using S = DecodeShape<DP, QR>;
  __shared__ DecodeShared<DP, QR> sh;
  __shared__ int row_count[kMaxRows], row_length[kMaxRows], row_splits[kMaxRows], row_first[kMaxRows + 1];
  __shared__ int row_page[kMaxRows];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int slot = lane / S::LPT, dc = lane % S::LPT;
  if (tid < c.B) {
    int count, length;
    capture_row(c, tid, count, length);
    row_count[tid] = count;
    row_length[tid] = length;
    row_splits[tid] = count == 0 ? 1 : (length + c.tok_item - 1) / c.tok_item;
    row_page[tid] = page_in_range(c.blocks ? c.blocks[(int64_t)tid * c.blocks_stride] : tid, c.B);
  }
  __syncthreads();
  if (tid == 0) {
    int first = 0;
    for (int r = 0; r < c.B; ++r) {
      row_first[r] = first;
      first += c.Hkv * row_splits[r];
    }
    row_first[c.B] = first;
  }
  __syncthreads();
  const int total = row_first[c.B];
  const DecodeParams p{c.q, c.k, c.v, c.out, c.o_sb, c.o_sh, c.o_st, c.part_o, c.part_ml, c.scale_log2, c.D, c.G, c.T};
  // One-round items: blocks take items blockIdx.x, blockIdx.x + gridDim.x, ...
  // Multi-round items: the grid covers every item of the capacity layout, one
  // block each (a loop would keep the next round's loads and the item state
  // live across iterations and double the registers).
  for (int item = blockIdx.x; item < total; item += (ROUNDS == 1 ? (int)gridDim.x : total)) {
    int r = 0;
    while (row_first[r + 1] <= item) ++r;
    RowSched rs;
    rs.batch = r;
    rs.count = row_count[r];
    rs.length = row_length[r];
    rs.item_begin = row_first[r];
    rs.nsplit = row_splits[r];
    rs.ntiles = 1;
    rs.rec_begin = (int64_t)r * c.row_records;
    DecodeItem it = locate_item(rs, item, ROUNDS * S::TOK_ROUND);
    it.kvb = row_page[r];
    DecodeRegs<DP, QR> regs;
    issue_item(p, it, regs, wave, slot, dc);
    process_item<DP, QR, ROUNDS>(p, it, regs, sh, wave, lane, slot, dc);
    if (ROUNDS > 1) break;
    __syncthreads();  // the next item reuses the block's reduction buffers
  }
}

template <int DP, int ROUNDS>
static hipError_t launch_decode_capture_r(const CaptureArgs &c, int qr, int blocks, hipStream_t stream) {
  switch (qr) {
    case 1: hipLaunchKernelGGL((decode_capture_kernel<DP, 1, ROUNDS>), dim3(blocks), dim3(256), 0, stream, c); break;
    case 2: hipLaunchKernelGGL((decode_capture_kernel<DP, 2, ROUNDS>), dim3(blocks), dim3(256), 0, stream, c); break;
    case 4: hipLaunchKernelGGL((decode_capture_kernel<DP, 4, ROUNDS>), dim3(blocks), dim3(256), 0, stream, c); break;
    default: hipLaunchKernelGGL((decode_capture_kernel<DP, 8, ROUNDS>), dim3(blocks), dim3(256), 0, stream, c); break;
  }
  return hipGetLastError();
}

hipError_t launch_decode_capture(const CaptureArgs &c, int dp, int qr, int rounds, int blocks, hipStream_t stream) {
  const bool multi = rounds == kDecodeRounds;
  switch (dp) {
    case 64: return multi ? launch_decode_capture_r<64, kDecodeRounds>(c, qr, blocks, stream)
                          : launch_decode_capture_r<64, 1>(c, qr, blocks, stream);
    case 128: return multi ? launch_decode_capture_r<128, kDecodeRounds>(c, qr, blocks, stream)
                           : launch_decode_capture_r<128, 1>(c, qr, blocks, stream);
    default: return multi ? launch_decode_capture_r<256, kDecodeRounds>(c, qr, blocks, stream)
                          : launch_decode_capture_r<256, 1>(c, qr, blocks, stream);
  }
}

int decode_tokens_per_item(int dp, int qr) {
  switch (dp * 16 + qr) {
#define XATTN_TOK(D, Q) \
  case D * 16 + Q: return DecodeShape<D, Q>::TOK_ROUND;
    XATTN_TOK(64, 1) XATTN_TOK(64, 2) XATTN_TOK(64, 4) XATTN_TOK(64, 8)
    XATTN_TOK(128, 1) XATTN_TOK(128, 2) XATTN_TOK(128, 4) XATTN_TOK(128, 8)
    XATTN_TOK(256, 1) XATTN_TOK(256, 2) XATTN_TOK(256, 4) XATTN_TOK(256, 8)
#undef XATTN_TOK
    default: return 0;
  }
}

template <int DP, int ROUNDS>
static hipError_t launch_decode_r(const AttnArgs &a, int qr, int blocks, hipStream_t stream) {
  switch (qr) {
    case 1: hipLaunchKernelGGL((decode_kernel<DP, 1, ROUNDS>), dim3(blocks), dim3(256), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((decode_kernel<DP, 2, ROUNDS>), dim3(blocks), dim3(256), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((decode_kernel<DP, 4, ROUNDS>), dim3(blocks), dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((decode_kernel<DP, 8, ROUNDS>), dim3(blocks), dim3(256), 0, stream, a); break;
  }
  return hipGetLastError();
}

template <int DP>
static hipError_t launch_decode_d(const AttnArgs &a, int qr, int rounds, int blocks, hipStream_t stream) {
  return rounds == kDecodeRounds ? launch_decode_r<DP, kDecodeRounds>(a, qr, blocks, stream)
                                 : launch_decode_r<DP, 1>(a, qr, blocks, stream);
}

// The XCC of each block of a small launch, for probe_xcd_dispatch.
constexpr int kXccProbeBlocks = 64;
__device__ uint32_t xcc_probe_ids[kXccProbeBlocks];

__global__ void __launch_bounds__(64) xcc_probe_kernel() {
  uint32_t xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  if (threadIdx.x == 0) xcc_probe_ids[blockIdx.x] = xcc & 15u;
}

hipError_t probe_xcd_dispatch(bool *round_robin, hipStream_t stream) {
  hipLaunchKernelGGL(xcc_probe_kernel, dim3(kXccProbeBlocks), dim3(64), 0, stream);
  hipError_t err = hipGetLastError();
  uint32_t ids[kXccProbeBlocks] = {};
  if (err == hipSuccess)
    err = hipMemcpyFromSymbolAsync(ids, HIP_SYMBOL(xcc_probe_ids), sizeof(ids), 0, hipMemcpyDeviceToHost, stream);
  if (err == hipSuccess) err = hipStreamSynchronize(stream);
  if (err != hipSuccess) return err;
  bool ok = true, distinct = false;
  for (int b = 8; b < kXccProbeBlocks; ++b) ok = ok && ids[b] == ids[b % 8];
  for (int b = 1; b < 8; ++b) distinct = distinct || ids[b] != ids[0];
  *round_robin = ok && distinct;
  return hipSuccess;
}

hipError_t launch_decode(const AttnArgs &a, int dp, int qr, int rounds, int blocks, hipStream_t stream) {
  switch (dp) {
    case 64: return launch_decode_d<64>(a, qr, rounds, blocks, stream);
    case 128: return launch_decode_d<128>(a, qr, rounds, blocks, stream);
    default: return launch_decode_d<256>(a, qr, rounds, blocks, stream);
  }
}

}  // namespace xattn
