// Chunked causal prefill attention on the gfx950 matrix cores (MFMA bf16),
// head dims up to 128 (padded to 64 or 128; head dim 256 is prefill_d256.hip).
//
// Replaces, for rows with more than 8 query vectors per KV head, the ATen
// FlashAttention-2 calls of compiler/common/kernels/attention.cpp:66-72 and
// :116-117.  Same math as decode.hip: lower-right causal softmax(scale*QK^T)V
// over the populated prefix, fp32 softmax state, bf16 in/out.
//
// Work item = (row, kv head, key split, tile of 128 query vectors).  The query
// vectors of one KV head are enumerated j = i*G + g (query i, grouped head g),
// so one tile serves all G heads that share the K/V tile in LDS.
//
// Waves: four query groups of 32 vectors x KH = 2: a block is 8 waves, two
// per SIMD, so one wave's MFMAs overlap the
// other's softmax; waves w and w+4 (the same SIMD) take alternate 64-key tiles
// of the item, each a whole tile, so a wave's per-tile softmax work (column
// max, rescale test and rescale) is spent once per 64 keys and its two 32-key
// score blocks are independent MFMA chains.  At the end waves w and w+4
// exchange halves of their accumulators and each finishes (and writes) half of
// the features.  Each wave computes the transposed problem with
// v_mfma_f32_32x32x16_bf16:
//   S^T[key, j]  = K[key, :] . Q[j, :]      A = K tile (LDS), B = Q^T (registers)
//   O^T[d, j]   += V^T[d, key] P^T[key, j]  A = V^T (LDS, transposing reads), B = P^T
// so a lane's accumulator column is one query vector: the online-softmax max /
// sum are per lane (plus one exchange with lane^32) and the S^T accumulator
// registers are directly the PV B operand.
//
// K/V tiles travel HBM -> LDS without registers: buffer_load_dwordx4 ... lds
// writes each lane's 16 bytes at M0 + 16 * lane, so every load instruction
// fills one contiguous 1 KB block, and the lanes choose which 16-byte chunks of
// the tile they fetch.  That choice implements an XOR swizzle of the chunks of
// each key row (against LDS bank conflicts) with no address arithmetic on the
// store side.  Tiles go through a ring of four stages in two-tile windows:
// while the window of tiles t, t+1 is computed, tiles t+2 and t+3 load.
//
// V is kept row-major ([key][d]) and read with ds_read_b64_tr_b16 (the
// transposing read of prefill_common.h), which gives the A-operand layout of
// the PV product.  The MFMA lane layouts are in prefill_common.h.
//
// Softmax rescaling is exact: whenever a tile raises a column's running max m,
// m becomes that tile max and the accumulator is rescaled (tiles that raise no
// column's max skip the rescale).  The key holding a column's maximum score
// then gets the weight exp2(0) = 1, exact in bf16.  A lazier rule (move m
// only when the tile max exceeds it by several log2 units) rounds that
// dominant weight to bf16 as well; on the 512-token chunk at offset 1536 it
// raised the worst output error from 7.5e-4 to 1.3e-3, above ATen
// FlashAttention's own bf16 error on the same inputs.
//
// Several splits of a tile write fp32 partial records, combined by merge.hip;
// a tile's records per split are laid out [D/4][128 vectors][4 features].
// The tile-0 / split-0 item zeroes the row's padded queries (t >= count).
#include "launch.h"
#include "prefill_common.h"

namespace xattn {

constexpr int kBN = 64;  // keys per LDS tile

// Head dims 64 and 128 (KH = 2: two waves per query group, 8 waves).
template <int DP, int KH>
struct PrefillShape {
  static_assert(DP <= 128 && KH == 2, "head dims 64 and 128; head dim 256 is prefill_d256.hip");
  static constexpr int THREADS = 256 * KH;
  static constexpr int NDS = DP / 16;                 // k-steps of the QK product
  static constexpr int NDT = DP / 32;                 // 32-row d tiles of the output
  static constexpr int CHUNKS = DP / 8;               // 16-byte chunks per key row
  static constexpr int BN = kBN;                      // keys per tile
  static constexpr int TILE = BN * DP;                // bf16 elements of one K (or V) tile
  static constexpr int LOADS = BN * CHUNKS / THREADS;  // 16-byte loads per thread per K (or V) tile
  // Two-tile windows over a ring of four stages (K+V of a tile: 4*TILE bytes).
  static constexpr int NST = 4;
  static_assert(NST * 4 * TILE <= 128 * 1024, "stages");
  // The two waves of a query group take alternate tiles, each all BN keys of its tile.
  static constexpr int KPW = BN;                      // keys of a tile each wave computes
  static constexpr int NKT = KPW / 32;                // 32-key sub-tiles per wave per tile
  static constexpr int HALF_T = NDT / 2;              // d tiles each wave finishes
  static constexpr int FOLD = 8 * (HALF_T * 16 + 2) * 64 * 4;  // bytes of the key-slice fold
  static constexpr int SMEM = NST * 4 * TILE > FOLD ? NST * 4 * TILE : FOLD;
};

// The kernel's body, shared by the launch with host-planned arguments
// (prefill_kernel) and the graph-capture launch that reads them from device
// memory (prefill_dev_kernel).
template <int DP, int KH, bool DEV>
__device__ __forceinline__ void prefill_body(const AttnArgs &a) {
  using S = PrefillShape<DP, KH>;
  constexpr int THREADS = S::THREADS, NDS = S::NDS, NDT = S::NDT, CHUNKS = S::CHUNKS;
  constexpr int TILE = S::TILE, LOADS = S::LOADS, NST = S::NST, KPW = S::KPW, NKT = S::NKT;
  static_assert(LOADS >= 1 && S::BN * CHUNKS == LOADS * THREADS, "tile = whole load instructions");
  __shared__ __attribute__((aligned(16))) uint16_t smem[S::SMEM / 2];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int col = lane & 31, half = lane >> 5;
  const int qgroup = wave & 3, khalf = wave >> 2;

  // The arguments the prologue needs, loaded in one round trip (see
  // XATTN_PIN_VIEW).  The output pointers and strides are read in the
  // epilogue instead: kept in SGPRs across the tile loop they cost more than
  // the late load.
  RowLookup<RowSched> rows;
  rows.load(a.rows);
  // The hardware hands consecutive blocks to the 8 XCDs in turn.  Block b
  // runs item xcd_begin[b % 8] + b / 8, so each XCD gets a contiguous run of
  // items, of about equal work; items are ordered (row, head, split, tile), so
  // the tiles that read the same keys share that XCD's L2.
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

  if (tile == 0 && split == 0 && cnt < T) zero_padded_queries(a, b, h, cnt, G, D, T, tid, THREADS);
  if constexpr (DEV) {
    if (cnt == 0) return;  // a row without queries (device-planned launches only): its zeros are written
  }

  // Key range of this tile and split.
  const int j_last = min(tile * kTileQ + kTileQ, qrows) - 1;
  const int kend = p0 + j_last / G + 1;
  int ks0, ks1;
  constexpr int BN = S::BN;
  split_range<BN>(kend, rs.nsplit, split, ks0, ks1);
  const int ntile = (ks1 - ks0 + BN - 1) / BN;

  // This lane's query vector.
  const int j = tile * kTileQ + qgroup * 32 + col;
  const bool jvalid = j < qrows;
  const int g = j % G, qi = j / G;
  const int lim = min(p0 + qi, ks1 - 1);  // last key this column may see in this split
  const int jw_first = tile * kTileQ + qgroup * 32;
  const bool wave_active = jw_first < qrows;
  const int wave_kmax = p0 + (min(jw_first + 31, qrows - 1)) / G;  // last key any column sees
  const int wave_kmin = p0 + jw_first / G;                          // last key of the first column

  // Tile loads.  Buffer descriptors end at the split's last key, so the rows
  // of a partial last tile read as zero (and are masked on the scores).  Load
  // i of this thread fills 16-byte slot q = (wave * LOADS + i) * 64 + lane of
  // the tile: key q / CHUNKS, slot q % CHUNKS, holding chunk slot ^ swizzle.
  // Chunks past D (padded head dims) repeat the row's last chunk: finite
  // values that only meet zero query features or unused output rows.
  // The K/V rows are read from row b's cache, or from its page when a page
  // table is given: the page is read once tiles 0 and 1 are loading from row
  // b, and another page (never with the identity table) reloads them.
  const uint32_t k_row = (uint32_t)kv.st * 2, v_row = (uint32_t)vv.st * 2;
  u32x4 k_rsrc = buffer_words(kv.p + b * kv.sb + (int64_t)h * kv.sh, (uint32_t)ks1 * k_row);
  u32x4 v_rsrc = buffer_words(vv.p + b * vv.sb + (int64_t)h * vv.sh, (uint32_t)ks1 * v_row);
  uint32_t k_voff[LOADS], v_voff[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; ++i) {
    const int q = (wave * LOADS + i) * 64 + lane;
    const int key = q / CHUNKS, slot = q % CHUNKS;
    k_voff[i] = key * k_row + (uint32_t)min(slot ^ k_swizzle<CHUNKS>(key), D / 8 - 1) * 16;
    v_voff[i] = key * v_row + (uint32_t)min(slot ^ v_swizzle<CHUNKS>(key), D / 8 - 1) * 16;
  }
  // The query tile goes through LDS the same way, into the last stage's
  // buffer, ahead of the first tiles: row jr = j - tile*kTileQ of the tile
  // holds query vector j, swizzled like K.  Rows past the tile's queries and
  // features past D load as zero (an offset past the descriptor's range).
  constexpr int QLOADS = kTileQ * CHUNKS / THREADS;
  static_assert(kTileQ * CHUNKS == QLOADS * THREADS && kTileQ * DP <= 2 * TILE, "query tile fits a stage");
  uint16_t *const qtile = smem + (NST - 1) * 2 * TILE;
  auto issue_query = [&]() {
    const u32x4 q_rsrc = buffer_words(qv.p + b * qv.sb + (int64_t)(h * G) * qv.sh, 0x7fffffffu);
    uint16_t *qdst = qtile;
#pragma unroll
    for (int i = 0; i < QLOADS; ++i) {
      const int qs = (wave * QLOADS + i) * 64 + lane;
      const int jr = qs / CHUNKS, chunk = (qs % CHUNKS) ^ k_swizzle<CHUNKS>(jr);
      const int jq = tile * kTileQ + jr;
      const uint32_t off = (jq < qrows && chunk < D / 8)
                               ? (uint32_t)(((jq % G) * qv.sh + (jq / G) * qv.st) * 2 + chunk * 16)
                               : 0x80000000u;
      lds_load16(q_rsrc, lds_address(qdst + (wave * QLOADS + i) * 512), off, 0);
    }
  };
  auto issue = [&](int stage, int kb) {
    uint16_t *kdst = smem + stage * 2 * TILE, *vdst = kdst + TILE;
#pragma unroll
    for (int i = 0; i < LOADS; ++i)
      lds_load16(k_rsrc, lds_address(kdst + (wave * LOADS + i) * 512), k_voff[i], (uint32_t)kb * k_row);
#pragma unroll
    for (int i = 0; i < LOADS; ++i)
      lds_load16(v_rsrc, lds_address(vdst + (wave * LOADS + i) * 512), v_voff[i], (uint32_t)kb * v_row);
  };

  // LDS read offsets (elements) of this lane, fixed for the whole item.
  // K (A operand of QK): key kl = 32kt + col, chunk 2ds + half.
  // Q (B operand, read once): row jr = qgroup*32 + col, same chunks.
  const int kl0 = col, jr0 = qgroup * 32 + col;
  int k_off[NDS];
#pragma unroll
  for (int ds = 0; ds < NDS; ++ds) k_off[ds] = kl0 * DP + (((2 * ds + half) ^ k_swizzle<CHUNKS>(kl0)) * 8);
  // V (A operand of PV) for d tile t: 16-lane group gq = lane/16, jj = lane%16
  // addresses key kv0 (+16hh +8 for the second read) and features
  // 32t + 16(gq%2) + 4(jj%4); kv0 % 4 == jj / 4 for every read.
  const int gq = lane >> 4, jj = lane & 15;
  const int kv0 = 4 * (gq >> 1) + (jj >> 2);
  int v_off[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t) {
    const int dch = 4 * t + 2 * (gq & 1) + ((jj & 3) >> 1);
    v_off[t] = kv0 * DP + ((dch ^ v_swizzle<CHUNKS>(kv0)) * 8) + 4 * (jj & 1);
  }

  f32x16 acc[NDT];
#pragma unroll
  for (int t = 0; t < NDT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[t][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const bf16x2 ones = as_bf16x2(0x3f803f80u);

  bf16x8 qf[NDS];  // Q^T B operands, read from LDS at tile 0
  auto compute = [&](int stage, int kb) {
    const uint16_t *Kt = smem + stage * 2 * TILE, *Vt = Kt + TILE;
    const int kw = kb;  // first key of this wave's tile
    if (!(wave_active && kw <= wave_kmax && kw < ks1)) return;
    f32x16 s[NKT];
    // The NKT 32-key blocks are independent accumulation chains; k-step
    // outer, so their MFMAs alternate.
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kt][r] = 0.0f;
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt) {
        const bf16x8 ka = as_bf16x8(*reinterpret_cast<const u32x4 *>(Kt + k_off[ds] + kt * 32 * DP));
        s[kt] = mfma32(ka, qf[ds], s[kt]);
      }
    // Mask keys past this column's causal limit or past the split.
    if (kw + KPW - 1 > wave_kmin || kw + KPW > ks1) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kw + kt * 32 + 8 * (r / 4) + 4 * half + (r % 4);
          s[kt][r] = key > lim ? -INFINITY : s[kt][r];
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kt][r]);
    const float mt = pair_max32(mx) * c;  // tile max of the column, log2 units
    if (__builtin_amdgcn_ballot_w64(mt > m_run)) {
      const float m_new = fmaxf(m_run, mt);
      const float alpha = fast_exp2(m_run - (m_new == -INFINITY ? 0.0f : m_new));
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] *= alpha;
      m_run = m_new;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    bf16x8 pb[NKT][2];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        u32x4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          typedef float f32x2 __attribute__((ext_vector_type(2)));
          const f32x2 pv = {fast_exp2(fmaf(s[kt][hh * 8 + 2 * e], c, -m_use)),
                            fast_exp2(fmaf(s[kt][hh * 8 + 2 * e + 1], c, -m_use))};
          const bf16x2 pk = __builtin_convertvector(pv, bf16x2);
          // The normaliser sums the bf16 weights the PV product uses, so the
          // output stays an exact convex combination of the values.
          l_run = __builtin_amdgcn_fdot2_f32_bf16(pk, ones, l_run, false);
          w[e] = __builtin_bit_cast(uint32_t, pk);
        }
        pb[kt][hh] = as_bf16x8(w);
      }
    // O^T += V^T P^T.  B element e of k-step (kt, hh) is S^T register hh*8+e:
    // key 32kt + 16hh + 8(e/4) + 4half + e%4, i.e. two runs of 4 keys, which the
    // two transposing reads of each A operand supply.
    // V operands one d tile ahead of their MFMAs (measured on cfg2, same
    // outputs: 21.2 against 21.5 us with the reads left to the scheduler;
    // K operands one k-step ahead in the score loop measured slower).
    u32x4 vop[2][NKT][2];
    auto vload = [&](int t, int buf) {
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const uint16_t *vp = Vt + v_off[t] + (kt * 32 + hh * 16) * DP;
          const u32x2 lo = lds_read_tr16(vp), hi = lds_read_tr16(vp + 8 * DP);
          vop[buf][kt][hh] = u32x4{lo.x, lo.y, hi.x, hi.y};
        }
    };
    vload(0, 0);
#pragma unroll
    for (int t = 0; t < NDT; ++t) {
      if (t + 1 < NDT) vload(t + 1, (t + 1) & 1);
#pragma unroll
      for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) acc[t] = mfma32(as_bf16x8(vop[t & 1][kt][hh]), pb[kt][hh], acc[t]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Pipeline.  The query tile is read into registers at tile 0, after which
  // a second barrier frees its buffer (the last stage).
  auto read_query = [&]() {
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
      qf[ds] = as_bf16x8(*reinterpret_cast<const u32x4 *>(qtile + jr0 * DP +
                                                           (((2 * ds + half) ^ k_swizzle<CHUNKS>(jr0)) * 8)));
    wait_lds_and_barrier();
  };
  {
    // Two-tile windows over four stages: at the start of the window of tiles
    // t, t+1 wait for their loads and synchronise (every wave is done with
    // tiles t-2 and t-1), refill those two stages with tiles t+2, t+3, then
    // compute: waves 0-3 tile t, waves 4-7 tile t+1, with no barrier between
    // the two, so the waves of a SIMD drift apart and overlap each other's
    // MFMA, LDS and softmax phases.
    const int raw_page = read_page(blocks, blocks_stride, b);
    __builtin_amdgcn_sched_barrier(0);
    if (ntile > 0) {
      issue_query();
      issue(0, ks0);
      if (ntile > 1) issue(1, ks0 + BN);
    }
    __builtin_amdgcn_sched_barrier(0);
    // Tiles 0 and 1 from the page, when it is not row b (block-uniform).
    const int page = page_in_range(raw_page, kv_rows);
    if (ntile > 0 && page != b) {
      wait_loads_and_barrier<0>();
      k_rsrc = buffer_words(kv.p + page * kv.sb + (int64_t)h * kv.sh, (uint32_t)ks1 * k_row);
      v_rsrc = buffer_words(vv.p + page * vv.sb + (int64_t)h * vv.sh, (uint32_t)ks1 * v_row);
      issue(0, ks0);
      if (ntile > 1) issue(1, ks0 + BN);
    }
    for (int t0 = 0; t0 < ntile; t0 += 4) {
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const int t = t0 + 2 * w;
        if (t < ntile) {
          wait_loads_and_barrier<0>();
          if (t == 0) read_query();
          if (t + 2 < ntile) issue((2 * w + 2) % 4, ks0 + (t + 2) * BN);
          if (t + 3 < ntile) issue((2 * w + 3) % 4, ks0 + (t + 3) * BN);
          if (khalf == 0) compute(2 * w, ks0 + t * BN);
          else if (t + 1 < ntile) compute(2 * w + 1, ks0 + (t + 1) * BN);
        }
      }
    }
  }

  // Per-lane partial sum -> column sum (lanes l and l^32 hold the two key halves of a 32x32 tile).
  l_run = pair_sum32(l_run);
  // Fold of the two waves' states.  Waves w and w+4 hold the same 32 query
  // vectors over alternate tiles; wave w finishes d tiles 0 .. NDT/2-1 and
  // wave w+4 the others:
  // each hands the other's half of its accumulator, and its (m, l), through
  // LDS, combines the half it keeps and writes that half of the output.
  constexpr int HALF_T = S::HALF_T;
  const int t_first = KH > 1 ? khalf * HALF_T : 0;  // first d tile this wave finishes
  if constexpr (KH > 1) {
    float(*xchg)[HALF_T * 16 + 2][64] = reinterpret_cast<float(*)[HALF_T * 16 + 2][64]>(smem);
    wait_loads_and_barrier<0>();  // every wave is done with the tiles
#pragma unroll
    for (int t = 0; t < NDT; ++t)
      if ((t < HALF_T) == (khalf == 1)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) xchg[wave][(t % HALF_T) * 16 + r][lane] = acc[t][r];
      }
    xchg[wave][HALF_T * 16][lane] = m_run;
    xchg[wave][HALF_T * 16 + 1][lane] = l_run;
    __syncthreads();
    const int partner = wave ^ 4;
    const float m_b = xchg[partner][HALF_T * 16][lane], l_b = xchg[partner][HALF_T * 16 + 1][lane];
    const float mx = fmaxf(m_run, m_b);
    const float mu = mx == -INFINITY ? 0.0f : mx;
    const float wa = fast_exp2(m_run - mu), wb = fast_exp2(m_b - mu);
#pragma unroll
    for (int t = 0; t < NDT; ++t)
      if ((t < HALF_T) == (khalf == 0)) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[t][r] = acc[t][r] * wa + xchg[partner][(t % HALF_T) * 16 + r][lane] * wb;
      }
    l_run = l_run * wa + l_b * wb;
    m_run = mx;
  }

  // Epilogue: d tiles t_first .. t_first + HALF_T - 1 of this wave.
  // acc[t][r] = O^T[d = 32t + 8(r/4) + 4half + r%4][column j].
  if (jvalid) {
    if (rs.nsplit == 1) {
      const float inv = 1.0f / l_run;
      uint16_t *dst = a.out + b * a.o_sb + (int64_t)(h * G + g) * a.o_sh + (int64_t)qi * a.o_st;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
        if (t >= t_first && t < t_first + HALF_T) {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int d = t * 32 + 8 * r4 + 4 * half;
            if (d < D)
              *reinterpret_cast<u32x2 *>(dst + d) =
                  u32x2{pack_bf16x2(acc[t][r4 * 4 + 0] * inv, acc[t][r4 * 4 + 1] * inv),
                        pack_bf16x2(acc[t][r4 * 4 + 2] * inv, acc[t][r4 * 4 + 3] * inv)};
          }
        }
    } else {
      // Record block of (head, split, tile): [D/4][kTileQ][4] floats, so a
      // store instruction writes two 512-byte runs of whole cache lines.  The
      // stores are non-temporal: the records stream out while the other items
      // still compute, instead of waiting in L2 for the write-back at the end
      // of the launch (the merge launch reads them back either way).
      const int jr = j - tile * kTileQ;
      const int64_t blk = rs.rec_begin + (((int64_t)h * rs.nsplit + split) * rs.ntiles + tile) * kTileQ;
      float *po = a.part_o + blk * D;
#pragma unroll
      for (int t = 0; t < NDT; ++t)
        if (t >= t_first && t < t_first + HALF_T) {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int d4 = 8 * t + 2 * r4 + half;  // features 4*d4 .. 4*d4+3
            if (d4 * 4 < D)
              __builtin_nontemporal_store(
                  f32x4{acc[t][r4 * 4 + 0], acc[t][r4 * 4 + 1], acc[t][r4 * 4 + 2], acc[t][r4 * 4 + 3]},
                  reinterpret_cast<f32x4 *>(po + (d4 * kTileQ + jr) * 4));
          }
        }
      if (half == 0 && khalf == 0)
        __builtin_nontemporal_store(u32x2{__float_as_uint(m_run), __float_as_uint(l_run)},
                                    reinterpret_cast<u32x2 *>(a.part_ml + 2 * (blk + jr)));
    }
  }
}

template <int DP, int KH>
__global__ void __launch_bounds__(256 * KH) prefill_kernel(const AttnArgs a) {
  prefill_body<DP, KH, false>(a);
}

template <int DP, int KH>
__global__ void __launch_bounds__(256 * KH) prefill_dev_kernel(const AttnArgs *__restrict__ a) {
  prefill_body<DP, KH, true>(*a);
}

// ceil(a / b) for 0 <= a, 0 < b < 2^31.
__device__ __forceinline__ int plan_ceil_div(int a, int b) {
  return (int)(((unsigned)a + (unsigned)b - 1u) / (unsigned)b);
}

// Inclusive prefix over the 64 lanes of the wave, in a fixed order.
template <typename V>
__device__ __forceinline__ V wave_inclusive_scan(V x, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d *= 2) {
    const V y = __shfl_up(x, d, 64);
    if (lane >= d) x += y;
  }
  return x;
}

__device__ __forceinline__ int read_lane(int x, int lane) { return __builtin_amdgcn_readlane(x, lane); }
__device__ __forceinline__ float read_lane(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}

constexpr int kPlanCandidates = kMaxRows * kMergeSerialSplits + 2;
constexpr int kPlanThreads = 1024;

// Graph-capture prefill plan: one block; its first wave holds one row per
// lane (B <= 64).
//  1. Lane r takes row r's count and length (capture_row) and its tiles of
//     128 query vectors, and estimates the 64-key tiles that all its tiles'
//     causal key ranges hold (a tile's splits together read its range once,
//     whatever the split size): tile t ends near key p0 + (t + 1) * 128 / G,
//     the last at the row's length, plus half a tile each for the partial
//     last 64 keys.
//  2. The split size.  Candidates are the host planner's range -- 256 to 2048
//     items' worth of keys, at least min_split_keys -- raised so that no row
//     takes more than splits_max splits, and within it every row's
//     split-count change points.  Each is priced, by a group of lanes with a
//     lane per row, as the larger of (work over 256 CUs + 3/4 of the longest
//     item) and the longest item, plus the records' trips and the merge
//     launch when a row splits, in the host planner's cost model (between the
//     list-scheduling bounds, where the host simulates the dispatch).  The
//     cheapest wins; ties go to the larger.
//  3. Rows' item, record and merge-vector offsets are wave prefix sums.  A
//     plan over items_max items (the limits make that impossible) would fall
//     back to unsplit rows, which always fit.
//  4. XCD runs of about equal work, as the host cuts them, with the cut inside
//     a (row, kv head) placed in proportion to its items, then clamped so that
//     no run exceeds run_max items.
// Writes *p.attn and *p.merge.
__global__ void __launch_bounds__(kPlanThreads) prefill_capture_plan_kernel(const PrefillPlanArgs p) {
  const CaptureArgs &c = p.c;
  __shared__ int4 s_row[kMaxRows];  // count, length, query tiles, key tiles (float bits)
  __shared__ int s_cand[kPlanCandidates];
  __shared__ int s_ncand;
  __shared__ unsigned long long s_best;
  const int tid = threadIdx.x, lane = tid & 63;
  const int B = c.B, G = c.G, Hkv = c.Hkv;
  const bool row_lane = tid < 64 && lane < B;
  int count = 0, length = 1, ntiles = 1;
  float kvtiles = 0.f;
  if (tid < 64) {
    if (row_lane) {
      capture_row(c, lane, count, length);
      if (count > 0) {
        ntiles = (count * G + kTileQ - 1) / kTileQ;
        const float m = (float)(ntiles - 1);
        kvtiles = (m * (float)(length - count) + (float)kTileQ / (float)G * m * (m + 1.f) * 0.5f + (float)length) *
                      (1.f / 64.f) + 0.5f * (float)ntiles;
      }
      s_row[lane] = make_int4(count, length, ntiles, __float_as_int(kvtiles));
    }
    // Keys of the rows with queries (host: choose_split_keys) and the longest row.
    int64_t keys = count > 0 ? (int64_t)Hkv * ntiles * length : 0;
    int longest_row = count > 0 ? length : 1;
#pragma unroll
    for (int d = 32; d >= 1; d /= 2) {
      keys += __shfl_xor(keys, d, 64);
      longest_row = max(longest_row, __shfl_xor(longest_row, d, 64));
    }
    auto keys_for = [&](int64_t target) {
      return max((int64_t)p.min_split_keys, ((keys + target - 1) / target + 63) / 64 * 64);
    };
    const int64_t floor_keys = (int64_t)plan_ceil_div(plan_ceil_div(longest_row, p.splits_max), 64) * 64;
    const int64_t lo64 = max(keys_for(2048), floor_keys), hi64 = max(keys_for(256), lo64);
    const int lo = (int)min<int64_t>(lo64, 0x7fffffff), hi = (int)min<int64_t>(hi64, 0x7fffffff);
    // Row lane r's change points: the smallest split (a multiple of 64) that
    // cuts it into n splits, for every n the range allows (n <= splits_max),
    // listed without gaps after those of the rows before it.
    int n = 1, n1 = 0;
    if (row_lane && count > 0) {
      n = max(1, plan_ceil_div(length, hi));
      n1 = min(plan_ceil_div(length, lo), p.splits_max);
    }
    int mine[kMergeSerialSplits], found = 0;
#pragma unroll
    for (int i = 0; i < kMergeSerialSplits; ++i, ++n) {
      const int k = n <= n1 ? max(p.min_split_keys, plan_ceil_div(plan_ceil_div(length, n), 64) * 64) : 0;
      mine[i] = k >= lo && k <= hi ? k : 0;
      found += mine[i] > 0;
    }
    const int listed = wave_inclusive_scan(found, lane);
    int at = 2 + listed - found;
#pragma unroll
    for (int i = 0; i < kMergeSerialSplits; ++i)
      if (mine[i] > 0) s_cand[at++] = mine[i];
    if (tid == 0) {
      s_cand[0] = lo;
      s_cand[1] = hi;
      s_ncand = 2 + read_lane(listed, 63);
      s_best = ~0ull;
    }
  }
  __syncthreads();
  // Thread t prices candidate t / R over row t % R, R the power of two at or
  // above B; the R lanes of a candidate then sum its work and records and
  // take its longest item.
  const int group = B <= 1 ? 1 : 1 << (32 - __clz(B - 1));
  const int ncand = s_ncand, per_pass = kPlanThreads / group;
  for (int base = 0; base < ncand; base += per_pass) {
    const int ci = base + tid / group, r = tid % group;
    const int k = ci < ncand ? s_cand[ci] : 0;
    float work = 0.f, longest = 0.f;
    int64_t records = 0;
    if (k > 0 && r < B) {
      const int4 row = s_row[r];
      if (row.x == 0) {
        work = (float)Hkv * p.item_us;
        longest = p.item_us;
      } else {
        const int L = row.y, nt = row.z;
        const int ns = plan_ceil_div(L, k);
        const int per = plan_ceil_div(plan_ceil_div(L, ns), 64) * 64;
        work = (float)Hkv * (__int_as_float(row.w) * p.tile_us + (float)(ns * nt) * p.item_us);
        longest = (float)plan_ceil_div(min(per, L), 64) * p.tile_us + p.item_us;
        records = ns > 1 ? (int64_t)Hkv * ns * nt * kTileQ : 0;
      }
    }
    for (int d = 1; d < group; d *= 2) {
      work += __shfl_xor(work, d, 64);
      longest = fmaxf(longest, __shfl_xor(longest, d, 64));
      records += __shfl_xor(records, d, 64);
    }
    if (k > 0 && r == 0) {
      const float us = fmaxf(work * (1.f / 256.f) + 0.75f * longest, longest) +
                       (records ? p.merge_us + (float)records * p.record_us : 0.f);
      atomicMin(&s_best, ((unsigned long long)__float_as_uint(us) << 32) | (unsigned)(0x7fffffff - k));
    }
  }
  __syncthreads();
  if (tid >= 64) return;
  const int split_keys = s_best == ~0ull ? 0x7fffffff : 0x7fffffff - (int)(uint32_t)s_best;
  int nsplit = count > 0 ? plan_ceil_div(length, split_keys) : 1;
  int items = row_lane ? Hkv * ntiles * nsplit : 0;
  int all_items = items;
#pragma unroll
  for (int d = 32; d >= 1; d /= 2) all_items += __shfl_xor(all_items, d, 64);
  if (all_items > p.items_max) {  // unreachable with the host's limits; unsplit rows fit
    nsplit = 1;
    items = row_lane ? Hkv * ntiles : 0;
  }
  const bool split = row_lane && nsplit > 1;
  const int records = split ? Hkv * nsplit * ntiles * kTileQ : 0;
  const int vectors = split ? Hkv * count * G : 0;
  const float work = row_lane ? (float)Hkv * (kvtiles * p.tile_us + (float)(nsplit * ntiles) * p.item_us) : 0.f;
  const int item_end = wave_inclusive_scan(items, lane), rec_end = wave_inclusive_scan(records, lane),
            vec_end = wave_inclusive_scan(vectors, lane), split_end = wave_inclusive_scan((int)split, lane);
  const float work_end = wave_inclusive_scan(work, lane);
  const int item_begin = item_end - items, rec_begin = rec_end - records;
  // Taken from the previous lane, so that the rows' work ranges tile exactly.
  const float work_before = __shfl_up(work_end, 1, 64), work_begin = lane == 0 ? 0.f : work_before;
  const int total_items = read_lane(item_end, 63), total_vectors = read_lane(vec_end, 63),
            split_rows = read_lane(split_end, 63);
  const float total_work = read_lane(work_end, 63);
  AttnArgs *const a = p.attn;
  MergeArgs *const m = p.merge;
  if (row_lane) {
    RowSched rs{};
    rs.batch = lane;
    rs.count = count;
    rs.length = length;
    rs.item_begin = item_begin;
    rs.nsplit = nsplit;
    rs.ntiles = ntiles;
    rs.rec_begin = rec_begin;
    a->rows[lane] = rs;
    if (split) {
      MergeRow mr{};
      mr.batch = lane;
      mr.count = count;
      mr.nsplit = nsplit;
      mr.item_begin = vec_end - vectors;
      mr.tiles = ntiles;
      mr.rec_begin = rec_begin;
      m->rows[split_end - 1] = mr;
    }
  }
  // XCD runs: cut x at x/8 of the work, inside the (row, kv head) that holds
  // it -- every lane places the cuts that fall in its row, then each cut is
  // read from the lane that holds it.
  int cut[9];
  cut[0] = 0;
  cut[8] = total_items;
#pragma unroll
  for (int x = 1; x < 8; ++x) {
    const float target = total_work * (float)x * 0.125f;
    const bool in = row_lane && work > 0.f && work_begin <= target && target < work_end;
    int mine = 0;
    if (in) {
      const int per_head = ntiles * nsplit;
      const float rel = (target - work_begin) / (work / (float)Hkv);
      const int h = min((int)rel, Hkv - 1);
      const int within = min((int)((rel - (float)h) * (float)per_head + 0.5f), per_head);
      mine = min(item_begin + h * per_head + within, total_items);
    }
    const unsigned long long holders = __ballot(in);
    cut[x] = holders ? read_lane(mine, __ffsll((long long)holders) - 1) : total_items;
  }
#pragma unroll
  for (int x = 1; x < 8; ++x)
    cut[x] = min(max(cut[x], max(cut[x - 1], total_items - (8 - x) * p.run_max)), cut[x - 1] + p.run_max);
  if (tid == 0) {
#pragma unroll
    for (int x = 0; x < 9; ++x) a->xcd_begin[x] = cut[x];
    a->q = c.q;
    a->k = c.k;
    a->v = c.v;
    a->out = c.out;
    a->o_sb = c.o_sb;
    a->o_sh = c.o_sh;
    a->o_st = c.o_st;
    a->part_o = c.part_o;
    a->part_ml = c.part_ml;
    a->scale_log2 = c.scale_log2;
    a->D = c.D;
    a->G = c.G;
    a->Hkv = c.Hkv;
    a->T = c.T;
    a->total_items = total_items;
    a->nrows = c.B;
    a->arrive_ctr = nullptr;
    a->tag = 0;
    a->blocks = c.blocks;
    a->blocks_stride = c.blocks_stride;
    a->kv_rows = c.B;
    m->out = c.out;
    m->o_sb = c.o_sb;
    m->o_sh = c.o_sh;
    m->o_st = c.o_st;
    m->part_o = c.part_o;
    m->part_ml = c.part_ml;
    m->D = c.D;
    m->G = c.G;
    m->total_items = total_vectors;
    m->nrows = split_rows;
  }
}

hipError_t launch_prefill_capture(const PrefillPlanArgs &p, int dp, unsigned blocks, hipStream_t stream) {
  hipLaunchKernelGGL(prefill_capture_plan_kernel, dim3(1), dim3(kPlanThreads), 0, stream, p);
  if (hipError_t err = hipGetLastError(); err != hipSuccess) return err;
  switch (dp) {
    case 64: hipLaunchKernelGGL((prefill_dev_kernel<64, 2>), dim3(blocks), dim3(512), 0, stream, p.attn); break;
    case 128: hipLaunchKernelGGL((prefill_dev_kernel<128, 2>), dim3(blocks), dim3(512), 0, stream, p.attn); break;
    default: return launch_prefill_d256_dev(p.attn, blocks, stream);
  }
  return hipGetLastError();
}

// Blocks per launch: 8 times the longest XCD run (blocks past their run exit
// at once).
hipError_t launch_prefill(const AttnArgs &a, int dp, hipStream_t stream) {
  int longest = 0;
  for (int x = 0; x < 8; ++x) {
    const int run = a.xcd_begin[x + 1] - a.xcd_begin[x];
    longest = run > longest ? run : longest;
  }
  const dim3 grid(8 * longest);
  switch (dp) {
    case 64: hipLaunchKernelGGL((prefill_kernel<64, 2>), grid, dim3(512), 0, stream, a); break;
    case 128: hipLaunchKernelGGL((prefill_kernel<128, 2>), grid, dim3(512), 0, stream, a); break;
    default: return launch_prefill_d256(a, grid.x, stream);
  }
  return hipGetLastError();
}

}  // namespace xattn
