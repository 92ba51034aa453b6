// Chunked causal prefill attention for head dims 129-256 (padded to 256) on
// the gfx950 matrix cores (MFMA bf16).
//
// Replaces, for rows with more than 8 query vectors per KV head, the ATen
// FlashAttention-2 calls of compiler/common/kernels/attention.cpp:66-72 and
// :116-117 (the Qwen3.5 full-attention layers: 16 query / 4 KV heads, head
// dim 256).  Same math as prefill.hip: lower-right causal softmax(scale*QK^T)V
// over the populated prefix, fp32 softmax state, bf16 in/out, the same work
// items (row, kv head, key split, tile of 128 query vectors j = i*G + g) and
// the same split records.
//
// Layout: 8 waves, two per SIMD, specialised.  Waves w < 4 (producers) and
// w + 4 (consumers) share a SIMD and query group w (32 query vectors):
//   * the producer computes, per 32-key tile, the scores S^T = K Q^T (16
//     chained 32x32x16 MFMAs over the 256 features, Q^T in registers), the
//     running max, the rescale factor and the bf16 weights P^T, and the
//     normaliser; it hands P^T and the factor to its consumer through LDS;
//   * the consumer keeps the 128 accumulator registers of O^T[256 x 32]: it
//     rescales them and accumulates V^T P^T (8 d tiles x 2 k-steps).
// Block-wide step s: the producer computes tile s (scores, then softmax), the
// consumer tile s-1 (rescale, then PV), so on each SIMD the producer's score
// MFMAs meet the consumer's rescale multiplies and the producer's softmax
// meets the consumer's PV MFMAs.  One barrier per step orders the hand-over
// (double-buffered) and the K/V rings.  Every value is computed with the
// instructions, operands and order of one wave doing a tile's scores,
// softmax and PV in turn: the same scores, maxima, weights, normaliser and
// accumulation, so the outputs do not depend on the split into two waves.
//
// Measured on cfg5 (ragged batch-8 prefill, 331 GFLOP): 466 us against
// 510 us for one wave per query group doing all of it (the same output
// bits).  s_memtime stamps per 32-key step: producer 1420 cycles of work,
// consumer 1450 (580 of them for the hand-over read), about 2000 with the
// barrier.  A variant whose producer issued the scores of tile s between the
// softmax instructions of tile s-1 (its MFMA chain hidden under its own VALU
// work, K and V in separate rings) took 512 us: the two waves of a SIMD then
// want both units at once instead of taking turns.
//
// K/V tiles travel HBM -> LDS through buffer_load ... lds over a ring of four
// 32 KB stages (K and V of a tile): tile t is read in steps t (K) and t+1
// (V), so step s issues the loads of tile s+2 into the stage of tile s-2.
#include "launch.h"
#include "prefill_common.h"

namespace xattn {

namespace {
constexpr int kDP = 256;
constexpr int kBN = 32;                           // keys per tile
constexpr int kChunks = kDP / 8;                  // 16-byte chunks per key row
constexpr int kTile = kBN * kDP;                  // bf16 elements of one K (or V) tile (16 KB)
constexpr int kThreads = 512;
constexpr int kLoads = kBN * kChunks / kThreads;  // 16-byte loads per thread per K (or V) tile
constexpr int kStages = 4;                        // stages of the K+V ring
constexpr int kSteps = kDP / 16;                  // k-steps of the scores
constexpr int kDTiles = kDP / 32;                 // 32-feature d tiles of the output
constexpr int kWeightsAt = 2 * kStages * kTile * 2;           // [2][4 groups][2][64 lanes] u32x4 weights
constexpr int kFactorAt = kWeightsAt + 2 * 4 * 2 * 64 * 16;   // [2][4 groups][64 lanes] f32 rescale factors
constexpr int kSmemBytes = kFactorAt + 2 * 4 * 64 * 4;
static_assert(kLoads * kThreads == kBN * kChunks, "tile = whole load instructions");
static_assert(kSmemBytes <= 160 * 1024, "LDS");
}  // namespace

// The kernel's body, shared by the launch with host-planned arguments and
// the graph-capture launch that reads them from device memory.
template <bool DEV>
__device__ __forceinline__ void prefill_d256_body(const AttnArgs &a) {
  __shared__ __attribute__((aligned(16))) uint16_t smem[kSmemBytes / 2];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;
  const int qgroup = wave & 3;
  const bool producer = wave < 4;

  // The arguments the prologue needs, in one round trip (see XATTN_PIN_VIEW).
  RowLookup<RowSched> rows;
  rows.load(a.rows);
  // Block b runs item xcd_begin[b % 8] + b / 8 (contiguous item runs per XCD,
  // so the tiles that read the same keys share an L2).
  const int xcd = (int)(blockIdx.x % 8);
  int run_begin = a.xcd_begin[xcd], run_end = a.xcd_begin[xcd + 1], nrows = a.nrows, G = a.G, D = a.D,
      T = a.T;
  float c = a.scale_log2;
  View qv = a.q, kv = a.k, vv = a.v;
  const int32_t *blocks = a.blocks;
  int64_t blocks_stride = a.blocks_stride;
  int kv_rows = a.kv_rows;
  asm volatile(""
               : XATTN_PIN_BEGINS(rows), XATTN_PIN_ROWSCHED(rows.first), "+s"(run_begin), "+s"(run_end),
                 "+s"(nrows), "+s"(G), "+s"(D), "+s"(T), "+s"(c), XATTN_PIN_VIEW(qv), XATTN_PIN_VIEW(kv),
                 XATTN_PIN_VIEW(vv), "+s"(blocks), "+s"(blocks_stride), "+s"(kv_rows));
  const int item = run_begin + (int)(blockIdx.x / 8);
  if (item >= run_end) return;
  const RowSched rs = rows.find(a.rows, nrows, item);
  const int local = item - rs.item_begin;
  const int per_head = rs.ntiles * rs.nsplit;
  const int h = local / per_head;
  const int split = (local - h * per_head) / rs.ntiles;
  const int tile = local - h * per_head - split * rs.ntiles;
  const int b = rs.batch, L = rs.length, cnt = rs.count;
  const int qrows = cnt * G, p0 = L - cnt;

  if (tile == 0 && split == 0 && cnt < T) zero_padded_queries(a, b, h, cnt, G, D, T, tid, kThreads);
  if constexpr (DEV) {
    if (cnt == 0) return;  // a row without queries (device-planned launches only): its zeros are written
  }

  // Key range of this tile and split.
  const int j_last = min(tile * kTileQ + kTileQ, qrows) - 1;
  const int kend = p0 + j_last / G + 1;
  int ks0, ks1;
  split_range<kBN>(kend, rs.nsplit, split, ks0, ks1);
  const int ntile = (ks1 - ks0 + kBN - 1) / kBN;

  // This lane's query vector (a producer and its consumer hold the same).
  const int j = tile * kTileQ + qgroup * 32 + col;
  const bool jvalid = j < qrows;
  const int g = j % G, qi = j / G;
  const int lim = min(p0 + qi, ks1 - 1);  // last key this column may see in this split
  const int jw_first = tile * kTileQ + qgroup * 32;
  const bool group_active = jw_first < qrows;
  const int group_kmax = p0 + (min(jw_first + 31, qrows - 1)) / G;  // last key any column sees
  const int group_kmin = p0 + jw_first / G;                          // last key of the first column
  // Whether tile t has keys some column of the group may see (uniform for the pair).
  auto tile_active = [&](int t) { return group_active && ks0 + t * kBN <= group_kmax; };

  // Tile loads (buffer descriptors end at the split's last key, so a partial
  // last tile reads as zero and is masked on the scores).  Load i of this
  // thread fills 16-byte slot q = (wave * kLoads + i) * 64 + lane of the tile:
  // key q / kChunks, slot q % kChunks, holding chunk slot ^ swizzle (clamped
  // into the row past D: finite values that meet zero query features or
  // unused output rows).  Every wave issues its share of every tile.
  // K/V rows of row b's cache, or of its page when a page table is given:
  // the page is read once tiles 0 and 1 are loading from row b, and another
  // page (never with the identity table) reloads them (prologue).
  const uint32_t k_row = (uint32_t)kv.st * 2, v_row = (uint32_t)vv.st * 2;
  u32x4 k_rsrc = buffer_words(kv.p + b * kv.sb + (int64_t)h * kv.sh, (uint32_t)ks1 * k_row);
  u32x4 v_rsrc = buffer_words(vv.p + b * vv.sb + (int64_t)h * vv.sh, (uint32_t)ks1 * v_row);
  uint32_t k_voff[kLoads], v_voff[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int q = (wave * kLoads + i) * 64 + lane;
    const int key = q / kChunks, slot = q % kChunks;
    k_voff[i] = key * k_row + (uint32_t)min(slot ^ k_swizzle<kChunks>(key), D / 8 - 1) * 16;
    v_voff[i] = key * v_row + (uint32_t)min(slot ^ v_swizzle<kChunks>(key), D / 8 - 1) * 16;
  }
  // Tile t (K, then V) goes to stage t % kStages.
  auto issue = [&](int t) {
    uint16_t *kdst = smem + (t % kStages) * 2 * kTile, *vdst = kdst + kTile;
    const int kb = ks0 + t * kBN;
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
      lds_load16(k_rsrc, lds_address(kdst + (wave * kLoads + i) * 512), k_voff[i], (uint32_t)kb * k_row);
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
      lds_load16(v_rsrc, lds_address(vdst + (wave * kLoads + i) * 512), v_voff[i], (uint32_t)kb * v_row);
  };
  // Start of step s: tile s+2 into the stage of tile s-2 (its K read in step
  // s-2, its V in step s-1).  End of step s: tile s+1 complete (only tile
  // s+2's loads may stay outstanding), the hand-over written, and the
  // buffers of step s-1 read.
  auto begin_step = [&](int step) {
    if (step + 2 < ntile) issue(step + 2);
  };
  auto end_step = [&](int step) {
    if (step + 2 < ntile) wait_loads_lds_and_barrier<2 * kLoads>();
    else wait_loads_lds_and_barrier<0>();
  };
  // Prologue: Q (producers), tiles 0 and 1; wait for Q and tile 0.
  auto prologue = [&]() {
    const int raw_page = read_page(blocks, blocks_stride, b);
    __builtin_amdgcn_sched_barrier(0);
    if (ntile > 0) issue(0);
    if (ntile > 1) issue(1);
    __builtin_amdgcn_sched_barrier(0);
    if (ntile > 1) wait_loads_and_barrier<2 * kLoads>();
    else wait_loads_and_barrier<0>();
    const int page = page_in_range(raw_page, kv_rows);
    if (page != b) {  // block-uniform: drain, then tiles 0 and 1 from the page
      wait_loads_and_barrier<0>();
      k_rsrc = buffer_words(kv.p + page * kv.sb + (int64_t)h * kv.sh, (uint32_t)ks1 * k_row);
      v_rsrc = buffer_words(vv.p + page * vv.sb + (int64_t)h * vv.sh, (uint32_t)ks1 * v_row);
      if (ntile > 0) issue(0);
      if (ntile > 1) issue(1);
      if (ntile > 1) wait_loads_and_barrier<2 * kLoads>();
      else wait_loads_and_barrier<0>();
    }
  };
  u32x4 *const wbuf = reinterpret_cast<u32x4 *>(reinterpret_cast<char *>(smem) + kWeightsAt);
  float *const fbuf = reinterpret_cast<float *>(reinterpret_cast<char *>(smem) + kFactorAt);
  float *const ml = fbuf;  // (m, l) hand-over at the end: the factor buffers are free then

  if (producer) {
    // Q^T B operands, straight from memory: k-step ks holds features
    // 16*ks + 8*half .. +7 of query vector j (zero past the row's queries and
    // past D).
    bf16x8 qf[kSteps];
    {
      const int jc = jvalid ? j : 0;
      const uint16_t *qrow = qv.p + b * qv.sb + (int64_t)(h * G + jc % G) * qv.sh + (int64_t)(jc / G) * qv.st;
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) {
        const int d0 = 16 * ks + 8 * half;
        const bool ok = jvalid && d0 < D;
        const u32x4 x = load16(qrow + (ok ? d0 : 0));
        qf[ks] = as_bf16x8(ok ? x : u32x4{0, 0, 0, 0});
      }
    }
    prologue();
    // K operand of k-step ds: key col, chunk 2ds + half.
    const int k_base = col * kDP, k_swz = k_swizzle<kChunks>(col);
    float m_run = -INFINITY, l_run = 0.0f;  // running max (log2 units) and normaliser of the column
    const bf16x2 ones = as_bf16x2(0x3f803f80u);
    for (int step = 0; step <= ntile; ++step) {
      begin_step(step);
      if (step < ntile && tile_active(step)) {
        const int kb = ks0 + step * kBN;
        const uint16_t *Kt = smem + (step % kStages) * 2 * kTile;
        // K operands in groups of two k-steps, one group ahead of the MFMAs.
        constexpr int GR = 2;
        u32x4 ka[2][GR];
        auto load = [&](int gi, int bi) {
#pragma unroll
          for (int u = 0; u < GR; ++u) {
            const int ds = gi * GR + u;
            ka[bi][u] = *reinterpret_cast<const u32x4 *>(Kt + k_base + (((2 * ds + half) ^ k_swz) * 8));
          }
        };
        f32x16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.0f;
        load(0, 0);
#pragma unroll
        for (int gi = 0; gi < kSteps / GR; ++gi) {
          if (gi + 1 < kSteps / GR) load(gi + 1, (gi + 1) & 1);
#pragma unroll
          for (int u = 0; u < GR; ++u) s = mfma32(as_bf16x8(ka[gi & 1][u]), qf[gi * GR + u], s);
          __builtin_amdgcn_sched_barrier(0);
        }
        // Mask keys past this column's causal limit or past the split.
        if (kb + kBN - 1 > group_kmin || kb + kBN > ks1) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int key = kb + 8 * (r / 4) + 4 * half + (r % 4);
            s[r] = key > lim ? -INFINITY : s[r];
          }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
        const float mt = pair_max32(mx) * c;  // tile max of the column, log2 units
        // The new running max and the rescale factor exp2(m_old - m_new):
        // exactly 1 for a column whose max stays (0 while no key of the
        // column has been visible: its state is still all zero).
        const float m_new = fmaxf(m_run, mt);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = fast_exp2(m_run - m_use);
        l_run *= alpha;
        m_run = m_new;
        const int buf = step & 1;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          u32x4 w;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            typedef float f32x2 __attribute__((ext_vector_type(2)));
            const f32x2 pv = {fast_exp2(fmaf(s[hh * 8 + 2 * e], c, -m_use)),
                              fast_exp2(fmaf(s[hh * 8 + 2 * e + 1], c, -m_use))};
            const bf16x2 pk = __builtin_convertvector(pv, bf16x2);
            // The normaliser sums the bf16 weights the PV product uses, so
            // the output stays an exact convex combination of the values.
            l_run = __builtin_amdgcn_fdot2_f32_bf16(pk, ones, l_run, false);
            w[e] = __builtin_bit_cast(uint32_t, pk);
          }
          wbuf[((buf * 4 + qgroup) * 2 + hh) * 64 + lane] = w;
        }
        fbuf[(buf * 4 + qgroup) * 64 + lane] = alpha;
      }
      end_step(step);
    }
    // Column sum: lanes l and l^32 hold the two key halves of each tile.
    // (m, l) go to the consumer, which writes the group's output.
    l_run = pair_sum32(l_run);
    ml[qgroup * 64 + lane] = m_run;
    ml[(4 + qgroup) * 64 + lane] = l_run;
    wait_lds_and_barrier();
    return;
  }

  // Consumer: O^T, acc[t][r] = O^T[d = 32t + 8(r/4) + 4half + r%4][column j].
  f32x16 acc[kDTiles];
#pragma unroll
  for (int t = 0; t < kDTiles; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
  prologue();
  // V operand of d tile t, k-step hh: 16-lane group gq = lane/16, jj =
  // lane%16 addresses key kv0 + 16hh (+8 for the second read) and features
  // 32t + 16(gq%2) + 4(jj%4); kv0 % 4 == jj / 4 for every read.
  const int gq = lane >> 4, jj = lane & 15;
  const int kv0 = 4 * (gq >> 1) + (jj >> 2);
  const int v_base = kv0 * kDP + 4 * (jj & 1), v_swz = v_swizzle<kChunks>(kv0);
  const int v_dch = 2 * (gq & 1) + ((jj & 3) >> 1);
  for (int step = 0; step <= ntile; ++step) {
    begin_step(step);
    if (step >= 1 && tile_active(step - 1)) {
      const int pbuf = (step - 1) & 1;
      const uint16_t *Vt = smem + ((step - 1) % kStages) * 2 * kTile + kTile;
      const float alpha = fbuf[(pbuf * 4 + qgroup) * 64 + lane];
      const bf16x8 pb[2] = {as_bf16x8(wbuf[((pbuf * 4 + qgroup) * 2 + 0) * 64 + lane]),
                            as_bf16x8(wbuf[((pbuf * 4 + qgroup) * 2 + 1) * 64 + lane])};
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
        for (int t = 0; t < kDTiles; ++t)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[t][r] *= alpha;
      }
      // O^T += V^T P^T.  B element e of k-step hh is S^T register 8hh + e:
      // key 16hh + 8(e/4) + 4half + e%4, i.e. two runs of 4 keys, which the
      // two transposing reads of each A operand supply.  V operands one d
      // tile ahead of their MFMAs.
      u32x4 va[2][2];
      auto vload = [&](int t, int bi) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const uint16_t *vp = Vt + v_base + (((4 * t + v_dch) ^ v_swz) * 8) + hh * 16 * kDP;
          const u32x2 lo = lds_read_tr16(vp), hi = lds_read_tr16(vp + 8 * kDP);
          va[bi][hh] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
      };
      vload(0, 0);
#pragma unroll
      for (int t = 0; t < kDTiles; ++t) {
        if (t + 1 < kDTiles) vload(t + 1, (t + 1) & 1);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) acc[t] = mfma32(as_bf16x8(va[t & 1][hh]), pb[hh], acc[t]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    end_step(step);
  }
  wait_lds_and_barrier();
  if (!jvalid) return;
  const float m_run = ml[qgroup * 64 + lane], l_run = ml[(4 + qgroup) * 64 + lane];
  if (rs.nsplit == 1) {
    const float inv = 1.0f / l_run;
    uint16_t *dst = a.out + b * a.o_sb + (int64_t)(h * G + g) * a.o_sh + (int64_t)qi * a.o_st;
#pragma unroll
    for (int t = 0; t < kDTiles; ++t)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d = t * 32 + 8 * r4 + 4 * half;
        if (d < D)
          *as_global(reinterpret_cast<u32x2 *>(dst + d)) =
              u32x2{pack_bf16x2(acc[t][r4 * 4 + 0] * inv, acc[t][r4 * 4 + 1] * inv),
                    pack_bf16x2(acc[t][r4 * 4 + 2] * inv, acc[t][r4 * 4 + 3] * inv)};
      }
  } else {
    // Record block of (head, split, tile): [D/4][kTileQ][4] floats (the
    // merge kernel's layout), written with non-temporal stores.
    const int jr = j - tile * kTileQ;
    const int64_t blk = rs.rec_begin + (((int64_t)h * rs.nsplit + split) * rs.ntiles + tile) * kTileQ;
    float *po = a.part_o + blk * D;
#pragma unroll
    for (int t = 0; t < kDTiles; ++t)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d4 = 8 * t + 2 * r4 + half;  // features 4*d4 .. 4*d4+3
        if (d4 * 4 < D)
          __builtin_nontemporal_store(
              f32x4{acc[t][r4 * 4 + 0], acc[t][r4 * 4 + 1], acc[t][r4 * 4 + 2], acc[t][r4 * 4 + 3]},
              as_global(reinterpret_cast<f32x4 *>(po + (d4 * kTileQ + jr) * 4)));
      }
    if (half == 0)
      __builtin_nontemporal_store(u32x2{__float_as_uint(m_run), __float_as_uint(l_run)},
                                  as_global(reinterpret_cast<u32x2 *>(a.part_ml + 2 * (blk + jr))));
  }
}

__global__ void __launch_bounds__(kThreads) prefill_d256_kernel(const AttnArgs a) { prefill_d256_body<false>(a); }

__global__ void __launch_bounds__(kThreads) prefill_d256_dev_kernel(const AttnArgs *__restrict__ a) {
  prefill_d256_body<true>(*a);
}

hipError_t launch_prefill_d256(const AttnArgs &a, unsigned blocks, hipStream_t stream) {
  hipLaunchKernelGGL(prefill_d256_kernel, dim3(blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_prefill_d256_dev(const AttnArgs *a, unsigned blocks, hipStream_t stream) {
  hipLaunchKernelGGL(prefill_d256_dev_kernel, dim3(blocks), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace xattn
