// Chunked causal prefill attention on the gfx950 matrix cores (MFMA bf16).
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
// Waves: four query groups of 32 vectors x KH.  With KH = 2 (head dims 64 and
// 128) a block is 8 waves, two per SIMD, so one wave's MFMAs overlap the
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
// store side.  NST tiles are in flight: while tile t is computed, the loads of
// tiles t+1 .. t+NST-1 are outstanding, with one barrier per tile.
//
// V is kept row-major ([key][d]) and read with ds_read_b64_tr_b16, which
// transposes 4x16 blocks of 16-bit elements within each 16-lane group: lane j
// supplies the address of V[k0 + j/4][d0 + 4(j%4) .. +3] and receives
// V[k0 .. k0+3][d0 + j], i.e. four consecutive keys of one feature, which is
// the A-operand layout of the PV product.
//
// MFMA 32x32x16 lane layout used (A: 32xK16, B: K16x32, C: 32x32):
//   A lane l: row l%32, k = 8*(l/32) + 0..7      B lane l: col l%32, same k
//   C lane l, reg r: row 8*(r/4) + 4*(l/32) + r%4, col l%32
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
#include "device_common.h"
#include "kernel_args.h"
#include "launch.h"

namespace xattn {

constexpr int kTileQ = 128;  // query vectors per work item
constexpr int kBN = 64;      // keys per LDS tile

typedef short shortx4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// Transposing 8-byte LDS read (see the header comment for the lane mapping).
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t *p) {
  const shortx4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) shortx4 *)(p));
  return __builtin_bit_cast(u32x2, r);
}

// One 16-byte-per-lane buffer load into LDS: lane i's 16 bytes land at LDS
// byte address m0 + 16 * i.  Written as inline asm so that the compiler does
// not track these loads: it would otherwise wait for all of them before any
// transposing LDS read, which would drain the load pipeline every tile.  The
// waits for them are explicit (wait_loads_and_barrier); loads the compiler
// does track are unaffected, since extra outstanding loads only make its own
// waits stricter.
__device__ __forceinline__ void lds_load16(u32x4 rsrc, uint32_t lds_byte, uint32_t voffset, uint32_t soffset) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(__builtin_amdgcn_readfirstlane(lds_byte)), "v"(voffset), "s"(rsrc),
                 "s"(__builtin_amdgcn_readfirstlane(soffset))
               : "memory", "m0");
}

// Buffer descriptor words for [base, base + bytes) (raw buffer, no stride;
// loads past `bytes` return zero).
__device__ __forceinline__ u32x4 buffer_words(const void *base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  return u32x4{(uint32_t)p, (uint32_t)(p >> 32) & 0xffffu, bytes, 0x00020000u};
}

__device__ __forceinline__ uint32_t lds_address(const uint16_t *p) {
  return (uint32_t)(uintptr_t)(lds_void *)(p);
}

// Wait until at most N vector-memory operations of this wave are outstanding
// (loads return in issue order), then synchronise the block.  The empty asm
// keeps the compiler from moving LDS accesses across the barrier.
template <int N>
__device__ __forceinline__ void wait_loads_and_barrier() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  // s_waitcnt encoding (gfx9): vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt_hi[15:14].
  __builtin_amdgcn_s_waitcnt((N & 15) | (0x7 << 4) | (0xF << 8));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Wait for this wave's LDS reads, then synchronise the block.
__device__ __forceinline__ void wait_lds_and_barrier() {
  __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Key range [ks0, ks1) of split `split` for a tile whose last visible key is kend-1.
template <int BN>
__device__ __forceinline__ void split_range(int kend, int nsplit, int split, int &ks0, int &ks1) {
  const int per = ((kend + nsplit - 1) / nsplit + BN - 1) / BN * BN;
  ks0 = min(kend, split * per);
  ks1 = min(kend, ks0 + per);
}

template <int DP, int KH>
struct PrefillShape {
  static constexpr int THREADS = 256 * KH;
  static constexpr int NDS = DP / 16;                 // k-steps of the QK product
  static constexpr int NDT = DP / 32;                 // 32-row d tiles of the output
  static constexpr int CHUNKS = DP / 8;               // 16-byte chunks per key row
  // D = 256 (one wave per SIMD, 128 accumulator registers, 32-key tiles)
  // stages the query tile in its own LDS region and keeps each wave's 64 Qᵀ
  // operand registers in AGPRs, which MFMA reads as its B operand directly
  // (the VGPRs hold the accumulators).
  static constexpr bool QLDS = DP == 256;
  static constexpr int BN = QLDS ? 32 : kBN;          // keys per tile
  static constexpr int TILE = BN * DP;                // bf16 elements of one K (or V) tile
  static constexpr int LOADS = BN * CHUNKS / THREADS;  // 16-byte loads per thread per K (or V) tile
  static constexpr int QBYTES = QLDS ? kTileQ * DP * 2 : 0;  // resident query tile
  // Tiles per barrier window (WIN) and LDS stages (K+V of a tile: 4*TILE
  // bytes): two-tile windows over a ring of four stages when it fits in
  // 128 KB, else one tile per barrier over a ring of as many stages as fit.
  static constexpr int WIN = !QLDS && 4 * TILE * 4 <= 128 * 1024 ? 2 : 1;
  static constexpr int NST = WIN == 2 ? 4 : (QLDS ? (160 * 1024 - QBYTES) / (4 * TILE) : (4 * TILE * 3 <= 100 * 1024 ? 3 : 2));
  // KH = 2: the two waves of a query group take alternate tiles (ALT), each
  // all BN keys of its tile.
  static constexpr bool ALT = KH > 1;
  static constexpr int KPW = ALT ? BN : BN / KH;      // keys of a tile each wave computes
  static constexpr int NKT = KPW / 32;                // 32-key sub-tiles per wave per tile
  static constexpr int HALF_T = KH > 1 ? NDT / 2 : NDT;  // d tiles each wave finishes
  static constexpr int FOLD = KH > 1 ? 8 * (HALF_T * 16 + 2) * 64 * 4 : 0;  // bytes of the key-slice fold
  static constexpr int SMEM = (NST * 4 * TILE + QBYTES > FOLD ? NST * 4 * TILE + QBYTES : FOLD);
};

// XOR swizzles of the 16-byte chunks of a key row (chunk c of key k is stored
// at slot c ^ swz(k)).  K: a K read takes chunk c of 32 consecutive keys, so
// the 16 keys served together land in 16 different slots.  V: the 32 lanes
// one LDS pass serves (8 bytes each) read chunks 4t .. 4t+3 of 4 consecutive
// keys (k0 % 4 == 0); the swizzle moves each key's four chunks to its own
// group of four slots, i.e. its own 16 of the 64 banks.  (With D = 64 two
// rows share the banks, so keys k and k+1 already differ in bank half.)
template <int CHUNKS>
__device__ __forceinline__ int k_swizzle(int key) { return key & (CHUNKS >= 16 ? 15 : CHUNKS - 1); }
template <int CHUNKS>
__device__ __forceinline__ int v_swizzle(int key) { return CHUNKS >= 16 ? 4 * (key & 3) : 4 * ((key >> 1) & 1); }

template <int DP, int KH>
__global__ void __launch_bounds__(256 * KH) prefill_kernel(const AttnArgs a) {
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
  asm volatile(""
               : XATTN_PIN_BEGINS(rows), XATTN_PIN_ROWSCHED(rows.first), "+s"(run_begin), "+s"(run_end),
                 "+s"(nrows), "+s"(G), "+s"(D), "+s"(T), "+s"(c), XATTN_PIN_VIEW(qv), XATTN_PIN_VIEW(kv),
                 XATTN_PIN_VIEW(vv));
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

  if (tile == 0 && split == 0 && cnt < T) {  // zero the row's padded queries
    const int chunks = D / 8, per = (T - cnt) * chunks;
    for (int idx = tid; idx < G * per; idx += THREADS) {
      const int g = idx / per, rest = idx - g * per;
      const int t = cnt + rest / chunks, ch = rest - (rest / chunks) * chunks;
      store16(a.out + b * a.o_sb + (int64_t)(h * G + g) * a.o_sh + (int64_t)t * a.o_st + ch * 8,
              u32x4{0, 0, 0, 0});
    }
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
  const uint32_t k_row = (uint32_t)kv.st * 2, v_row = (uint32_t)vv.st * 2;
  const u32x4 k_rsrc = buffer_words(kv.p + b * kv.sb + (int64_t)h * kv.sh, (uint32_t)ks1 * k_row);
  const u32x4 v_rsrc = buffer_words(vv.p + b * vv.sb + (int64_t)h * vv.sh, (uint32_t)ks1 * v_row);
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
  static_assert(kTileQ * CHUNKS == QLOADS * THREADS && (S::QLDS || kTileQ * DP <= 2 * TILE),
                "query tile fits a stage");
  uint16_t *const qtile = smem + (S::QLDS ? NST * 2 * TILE : (NST - 1) * 2 * TILE);
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
  // K (A operand of QK): key kl = kbase + 32kt + col, chunk 2ds + half, with
  // kbase the first key of the wave's share of a tile (0 when the waves of a
  // query group alternate tiles).
  // Q (B operand, read once): row jr = qgroup*32 + col, same chunks.
  const int kbase = S::ALT ? 0 : khalf * KPW;
  const int kl0 = kbase + col, jr0 = qgroup * 32 + col;
  int k_off[NDS];
#pragma unroll
  for (int ds = 0; ds < NDS; ++ds) k_off[ds] = kl0 * DP + (((2 * ds + half) ^ k_swizzle<CHUNKS>(kl0)) * 8);
  // V (A operand of PV) for d tile t: 16-lane group gq = lane/16, jj = lane%16
  // addresses key kv0 (+16hh +8 for the second read) and features
  // 32t + 16(gq%2) + 4(jj%4); kv0 % 4 == jj / 4 for every read.
  const int gq = lane >> 4, jj = lane & 15;
  const int kv0 = kbase + 4 * (gq >> 1) + (jj >> 2);
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
    const int kw = kb + kbase;  // first key of this wave's share
    if (!(wave_active && kw <= wave_kmax && kw < ks1)) return;
    f32x16 s[NKT];
    if constexpr (S::QLDS) {
      // Qᵀ operands from AGPRs (read at tile 0); K operands from LDS in groups
      // of two k-steps, one group ahead of the MFMAs, and the scheduler may
      // not hoist further: the 128 accumulator registers leave no room for
      // more.  Measured on cfg5: 546.8 -> 539.2 us against Qᵀ read from LDS
      // next to each K operand (a third of the tile's LDS reads).
      static_assert(KH == 1 && NKT == 1, "D = 256 layout: one key slice of 32-key tiles");
      constexpr int GR = 2;
      u32x4 ka[2][GR];
      auto load = [&](int g, int buf) {
#pragma unroll
        for (int u = 0; u < GR; ++u) ka[buf][u] = *reinterpret_cast<const u32x4 *>(Kt + k_off[g * GR + u]);
      };
#pragma unroll
      for (int r = 0; r < 16; ++r) s[0][r] = 0.0f;
      load(0, 0);
#pragma unroll
      for (int g = 0; g < NDS / GR; ++g) {
        if (g + 1 < NDS / GR) load(g + 1, (g + 1) & 1);
#pragma unroll
        for (int u = 0; u < GR; ++u) s[0] = mfma32(as_bf16x8(ka[g & 1][u]), qf[g * GR + u], s[0]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
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
    if constexpr (S::QLDS) {
      // V operands one d tile ahead of its MFMAs.  Measured on cfg5 (same
      // outputs): groups of one d tile 504 us, of two 516 us, of four 503 us,
      // all eight at once 526 us.
      constexpr int GT = 1;
      u32x4 va[2][GT][2];
      auto load = [&](int g, int buf) {
#pragma unroll
        for (int u = 0; u < GT; ++u)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const uint16_t *vp = Vt + v_off[g * GT + u] + hh * 16 * DP;
            const u32x2 lo = lds_read_tr16(vp), hi = lds_read_tr16(vp + 8 * DP);
            va[buf][u][hh] = u32x4{lo.x, lo.y, hi.x, hi.y};
          }
      };
      load(0, 0);
#pragma unroll
      for (int g = 0; g < NDT / GT; ++g) {
        if (g + 1 < NDT / GT) load(g + 1, (g + 1) & 1);
#pragma unroll
        for (int u = 0; u < GT; ++u)
#pragma unroll
          for (int hh = 0; hh < 2; ++hh)
            acc[g * GT + u] = mfma32(as_bf16x8(va[g & 1][u][hh]), pb[0][hh], acc[g * GT + u]);
        __builtin_amdgcn_sched_barrier(0);
      }
      return;
    }
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
  constexpr int PER_TILE = 2 * LOADS;  // load instructions per tile per thread
  auto read_query = [&]() {
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds)
      qf[ds] = as_bf16x8(*reinterpret_cast<const u32x4 *>(qtile + jr0 * DP +
                                                           (((2 * ds + half) ^ k_swizzle<CHUNKS>(jr0)) * 8)));
    if constexpr (S::QLDS) {
      // One wave per SIMD leaves the AGPRs free: the Qᵀ operands live there
      // for the item (MFMA reads its B operand from AGPRs directly).
#pragma unroll
      for (int ds = 0; ds < NDS; ++ds) asm volatile("" : "+a"(qf[ds]));
    }
    wait_lds_and_barrier();
  };
  if constexpr (S::WIN == 2) {
    // Two-tile windows over four stages: at the start of the window of tiles
    // t, t+1 wait for their loads and synchronise (every wave is done with
    // tiles t-2 and t-1), refill those two stages with tiles t+2, t+3, then
    // compute: waves 0-3 tile t, waves 4-7 tile t+1, with no barrier between
    // the two, so the waves of a SIMD drift apart and overlap each other's
    // MFMA, LDS and softmax phases.
    if (ntile > 0) {
      issue_query();
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
          static_assert(S::ALT, "two-tile windows: the waves of a query group alternate tiles");
          if (khalf == 0) compute(2 * w, ks0 + t * BN);
          else if (t + 1 < ntile) compute(2 * w + 1, ks0 + (t + 1) * BN);
        }
      }
    }
  } else {
    // One tile per barrier: before computing tile t, wait for its loads (the
    // loads of tiles t+1 .. t+NST-2 may stay outstanding), barrier (the tile
    // is complete in LDS and every wave has finished tile t-1), then refill
    // the stage of tile t-1 with tile t+NST-1.
    if (ntile > 0) {
      issue_query();
#pragma unroll
      for (int st = 0; st < NST - 1; ++st)
        if (st < ntile) issue(st, ks0 + st * BN);
    }
    for (int t0 = 0; t0 < ntile; t0 += NST) {
#pragma unroll
      for (int st = 0; st < NST; ++st) {
        const int t = t0 + st;
        if (t < ntile) {
          const int ahead = min(ntile - 1 - t, NST - 2);  // tiles after t already issued
          if constexpr (NST == 3) {
            if (ahead >= 1) wait_loads_and_barrier<PER_TILE>();
            else wait_loads_and_barrier<0>();
          } else {
            wait_loads_and_barrier<0>();
          }
          if (t == 0) read_query();
          if (t + NST - 1 < ntile) issue((st + NST - 1) % NST, ks0 + (t + NST - 1) * BN);
          compute(st, ks0 + t * BN);
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

// The D = 256 kernel is built in its own translation unit (prefill_d256.hip
// includes this file with XATTN_PREFILL_D256 defined), so that it can take
// its own scheduler flags.
#ifdef XATTN_PREFILL_D256
hipError_t launch_prefill_d256(const AttnArgs &a, unsigned blocks, hipStream_t stream) {
  hipLaunchKernelGGL((prefill_kernel<256, 1>), dim3(blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}
#else
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
#endif

}  // namespace xattn
