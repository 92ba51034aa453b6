// Merge of split-KV partial records into the bf16 output.
//
// When the keys of a group of query vectors are split over several work
// items, each item writes, per query vector, an fp32 record: unnormalised
// output o[D] and the pair (m, l) -- running max in log2 units and sum.  This
// kernel combines the records of one query vector:
//   M = max_s m_s,  w_s = exp2(m_s - M),  out = sum_s w_s o_s / sum_s w_s l_s
// Each thread folds its share of the splits with an online rescale (running
// max, sum and accumulator), in increasing split order; thread states are then
// folded in a fixed order, so the result is deterministic.  Splits that saw no
// visible key carry m = -inf and weight 0.  Running as its own launch, it reads
// the records after the producing kernel has completed, which orders them
// without any device-scope fence inside the attention kernels.
//
// With few splits per vector (prefill, short decode rows) a 256-thread block
// (512 for D = 256) holds VPB query vectors x FC feature lanes (4 features
// each), one thread owning a vector's 4 features across all splits.  With
// many splits (long
// decode rows) a block holds FS feature lanes of one vector and SG = THREADS /
// FS split lanes: all FC feature lanes up to kMergeSliceSplits splits, past
// that a slice of them, the FC / FS slices of a vector being separate blocks,
// so a very long row's records are read by many CUs at once.  THREADS (256 to
// 1024) is chosen so that a lane loads at most one batch of 16 records.
//
// Blocks are dealt to the 8 XCDs in contiguous runs of work groups (block b
// runs group (b % 8) * (grid / 8) + b / 8), the order the prefill kernel
// gives its items, so the records a head's tiles wrote through one XCD's L2
// are mostly read back on that XCD, and a vector's slices share the (m, l)
// reads in one L2.
#include "device_common.h"
#include "kernel_args.h"
#include "launch.h"

namespace xattn {

// Query vectors per prefill record block (the prefill kernel's query tile).
constexpr int kMergeTile = 128;

struct MergeState {
  float m, l;
  f32x4 o;
};

__device__ __forceinline__ void fold(MergeState &st, float ms, float ls, f32x4 os) {
  if (ms == -INFINITY) return;
  const float mn = fmaxf(st.m, ms);
  const float a = fast_exp2(st.m - mn), w = fast_exp2(ms - mn);  // st.m = -inf -> a = 0
  st.l = st.l * a + ls * w;
  st.o.x = st.o.x * a + os.x * w;
  st.o.y = st.o.y * a + os.y * w;
  st.o.z = st.o.z * a + os.z * w;
  st.o.w = st.o.w * a + os.w * w;
  st.m = mn;
}

// LDS states of a block with SG > 1 split lanes over FS feature lanes.
template <int FS, int SG>
using MergeRed = MergeState[SG > 1 ? SG : 1][SG > 1 ? FS : 1];

// Folds the nsplit records of one query vector over this thread's 4 features
// and writes them as bf16 at dst.  Record s: o at part_o + o_base + s * o_step,
// (m, l) at part_ml + 2 * (ml_base + s * ml_step).  With SG > 1 split lanes
// per feature group every thread of the block must call it (it synchronises
// the block); `active` is false for threads past the vectors or features, and
// f is the thread's feature lane within the block's FS.  Every record of a
// batch is loaded before any is folded: a lane's splits take
// ceil(nsplit / (SG * INFLIGHT)) memory round trips.
template <int FS, int SG>
__device__ __forceinline__ void fold_and_write(MergeRed<FS, SG> &red, const float *part_o, const float *part_ml,
                                               int64_t o_base, int64_t o_step, int64_t ml_base, int64_t ml_step,
                                               int nsplit, bool active, int sg, int f, uint16_t *dst) {
  constexpr int INFLIGHT = SG > 1 ? 16 : 4;
  MergeState st{-INFINITY, 0.0f, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
  if (active) {
    for (int s0 = sg; s0 < nsplit; s0 += INFLIGHT * SG) {
      u32x2 ml[INFLIGHT];
      f32x4 o[INFLIGHT];
#pragma unroll
      for (int u = 0; u < INFLIGHT; ++u)
        if (s0 + u * SG < nsplit) {  // a lane loads only its own splits' records
          const int64_t sp = s0 + u * SG;
          ml[u] = *as_global(reinterpret_cast<const u32x2 *>(part_ml + 2 * (ml_base + sp * ml_step)));
          o[u] = *as_global(reinterpret_cast<const f32x4 *>(part_o + o_base + sp * o_step));
        }
#pragma unroll
      for (int u = 0; u < INFLIGHT; ++u)
        if (s0 + u * SG < nsplit) fold(st, __uint_as_float(ml[u].x), __uint_as_float(ml[u].y), o[u]);
    }
  }
  if constexpr (SG > 1) {
    red[sg][f] = st;
    __syncthreads();
    if (sg != 0) return;
    // The states are read eight at a time before they are folded (in split
    // lane order), so the fold waits for one LDS round trip per eight lanes.
    for (int k0 = 1; k0 < SG; k0 += 8) {
      MergeState other[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k0 + u < SG) other[u] = red[k0 + u][f];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k0 + u < SG) fold(st, other[u].m, other[u].l, other[u].o);
    }
  }
  if (!active) return;
  const float inv = 1.0f / st.l;
  *as_global(reinterpret_cast<u32x2 *>(dst)) =
      u32x2{pack_bf16x2(st.o.x * inv, st.o.y * inv), pack_bf16x2(st.o.z * inv, st.o.w * inv)};
}

// The kernel's body, shared by the launch with host-planned arguments
// (merge_kernel) and the graph-capture launch that reads them from device
// memory (merge_dev_kernel).
template <int DP, int SG, int THREADS, int FS, bool DEV>
__device__ __forceinline__ void merge_body(const MergeArgs &a) {
  constexpr int FC = DP / 4;                         // feature lanes of a vector
  static_assert(SG == 1 ? FS == FC : FS * SG == THREADS, "block shape");
  constexpr int NS = FC / FS;                        // feature slices per vector (SG > 1)
  constexpr int VPB = SG > 1 ? 1 : THREADS / FC;     // query vectors per block
  __shared__ MergeRed<FS, SG> red;

  // Few splits: vectors vary fastest across a block's threads (the prefill
  // record layout keeps a tile's vectors contiguous per feature group).
  // Many splits: the slice's feature lanes vary fastest.
  const int tid = threadIdx.x;
  const int fl = SG > 1 ? tid % FS : tid / VPB, sg = SG > 1 ? tid / FS : 0;
  const int vl = VPB == 1 ? 0 : tid % VPB;
  // Every argument of the block, loaded in one round trip (see XATTN_PIN_VIEW).
  RowLookup<MergeRow> rows;
  rows.load(a.rows);
  int total_items = a.total_items, nrows = a.nrows, D = a.D, G = a.G;
  uint16_t *out = a.out;
  int64_t o_sb = a.o_sb, o_sh = a.o_sh, o_st = a.o_st;
  const float *part_o = a.part_o, *part_ml = a.part_ml;
  asm volatile(""
               : XATTN_PIN_BEGINS(rows), XATTN_PIN_MERGEROW(rows.first), "+s"(total_items), "+s"(nrows), "+s"(D),
                 "+s"(G), "+s"(out), "+s"(o_sb), "+s"(o_sh), "+s"(o_st), "+s"(part_o), "+s"(part_ml));
  // Work groups: VPB vectors (few splits) or one slice of one vector.  The
  // grid is the groups rounded up to a multiple of 8 (launch_merge_d).
  const int groups = SG > 1 ? total_items * NS : (total_items + VPB - 1) / VPB;
  // A grid sized for more groups (device-planned launches) leaves surplus blocks.
  if constexpr (DEV) {
    if ((int)(blockIdx.x / 8) >= (groups + 7) / 8) return;
  }
  const int group = (int)(blockIdx.x % 8) * ((groups + 7) / 8) + (int)(blockIdx.x / 8);
  const int vec = SG > 1 ? group / NS : group * VPB + vl;
  const int f = SG > 1 ? (group - vec * NS) * FS + fl : fl;  // feature lane of the vector
  const bool vvalid = vec < total_items;
  const MergeRow mr = rows.find(a.rows, nrows, vvalid ? vec : 0);
  const int local = vec - mr.item_begin;
  const int qrows = mr.count * G;
  const int h = local / qrows, j = local - h * qrows;
  const int d = f * 4;
  // Record s of this vector: o at part_o + o_base + s * o_step, (m, l) at
  // part_ml + 2 * (ml_base + s * ml_step).
  int64_t o_base, o_step, ml_base, ml_step;
  if (mr.tiles == 0) {
    ml_base = mr.rec_begin + (int64_t)h * mr.nsplit * qrows + j;
    ml_step = qrows;
    o_base = ml_base * D + d;
    o_step = ml_step * D;
  } else {
    const int tile = j / kMergeTile, jr = j - tile * kMergeTile;
    const int64_t blk = mr.rec_begin + ((int64_t)h * mr.nsplit * mr.tiles + tile) * kMergeTile;
    ml_base = blk + jr;
    ml_step = (int64_t)mr.tiles * kMergeTile;
    o_base = blk * D + (f * kMergeTile + jr) * 4;
    o_step = ml_step * D;
  }

  const int g = j % G, i = j / G;
  fold_and_write<FS, SG>(red, part_o, part_ml, o_base, o_step, ml_base, ml_step, mr.nsplit, vvalid && d < D, sg, fl,
                         out + mr.batch * o_sb + (int64_t)(h * G + g) * o_sh + (int64_t)i * o_st + d);
}

// Feature lanes per block past kMergeSliceSplits splits: 64 features, 256
// contiguous bytes of each record.  Measured on MI355X: slicing takes a
// 16384-key D = 256 row's merge from 10.3 to 7.2 us at 256 splits and from
// 6.5 to 5.9 us at 128, and makes merges of 17 to 52 splits 0.2-0.8 us
// slower than one block per vector.
constexpr int kMergeSliceLanes = 16;
constexpr int kMergeSliceSplits = 64;

template <int DP, int SG, int THREADS, int FS>
__global__ void __launch_bounds__(THREADS) merge_kernel(const MergeArgs a) {
  merge_body<DP, SG, THREADS, FS, false>(a);
}

template <int DP, int SG, int THREADS, int FS>
__global__ void __launch_bounds__(THREADS) merge_dev_kernel(const MergeArgs *__restrict__ a) {
  merge_body<DP, SG, THREADS, FS, true>(*a);
}

// The merge's launch: host arguments `a`, or (DEV) the arguments at `dev`;
// the grid covers `vectors` query vectors.
template <int DP, int SG, int THREADS, int FS, bool DEV>
static void launch_merge_kernel(dim3 grid, const MergeArgs &a, const MergeArgs *dev, hipStream_t stream) {
  if constexpr (DEV)
    hipLaunchKernelGGL((merge_dev_kernel<DP, SG, THREADS, FS>), grid, dim3(THREADS), 0, stream, dev);
  else
    hipLaunchKernelGGL((merge_kernel<DP, SG, THREADS, FS>), grid, dim3(THREADS), 0, stream, a);
}

template <int DP, bool DEV>
static hipError_t launch_merge_d(const MergeArgs &a, const MergeArgs *dev, int max_splits, int64_t vectors,
                                 hipStream_t stream) {
  constexpr int FC = DP / 4;
  // Grids are rounded up to a multiple of the 8 XCDs; surplus groups exit.
  if (max_splits <= kMergeSerialSplits) {
    // 8 vectors per block for D = 256 (512 threads), so that a wave's load
    // reads whole 128-byte lines of the prefill record layout (cfg5's merge
    // 3 us faster than with 4 vectors and half lines; same outputs).
    constexpr int THREADS = DP == 256 ? 512 : 256;
    constexpr int VPB = THREADS / FC;
    launch_merge_kernel<DP, 1, THREADS, FC, DEV>(dim3(((vectors + VPB - 1) / VPB + 7) / 8 * 8), a, dev, stream);
  } else if (max_splits <= kMergeSliceSplits) {
    // One block per vector, with enough split lanes that each lane loads at
    // most one batch of 16 records when the block can grow to 1024 threads.
    const dim3 grid((vectors + 7) / 8 * 8);
    if (max_splits <= 16 * (256 / FC))
      launch_merge_kernel<DP, 256 / FC, 256, FC, DEV>(grid, a, dev, stream);
    else if (max_splits <= 16 * (512 / FC))
      launch_merge_kernel<DP, 512 / FC, 512, FC, DEV>(grid, a, dev, stream);
    else
      launch_merge_kernel<DP, 1024 / FC, 1024, FC, DEV>(grid, a, dev, stream);
  } else {
    // One block per (vector, slice of FS feature lanes).
    constexpr int FS = FC < kMergeSliceLanes ? FC : kMergeSliceLanes;
    const dim3 grid((vectors * (FC / FS) + 7) / 8 * 8);
    if (max_splits <= 16 * (256 / FS))
      launch_merge_kernel<DP, 256 / FS, 256, FS, DEV>(grid, a, dev, stream);
    else
      launch_merge_kernel<DP, 512 / FS, 512, FS, DEV>(grid, a, dev, stream);
  }
  return hipGetLastError();
}

// Graph-capture merge: one block per query vector of the capacity layout
// (row, kv head, vector j < T * G), with split lanes over the splits.  The
// row's count and length come from the device offsets; vectors past the row's
// queries and rows whose keys fit one item (written by the decode kernel
// directly) have nothing to merge.
template <int DP, int SG, int THREADS>
__global__ void __launch_bounds__(THREADS) merge_capture_kernel(const CaptureArgs c) {
  constexpr int FC = DP / 4;
  static_assert(THREADS == FC * SG, "one query vector per block");
  __shared__ MergeRed<FC, SG> red;
  const int tid = threadIdx.x, f = tid % FC, sg = tid / FC;
  const int per_row = c.Hkv * c.T * c.G;
  const int r = (int)blockIdx.x / per_row, local = (int)blockIdx.x - r * per_row;
  const int qv_max = c.T * c.G;
  const int h = local / qv_max, j = local - h * qv_max;
  int count, length;
  capture_row(c, r, count, length);
  const int qrows = count * c.G;
  const int nsplit = (length + c.tok_item - 1) / c.tok_item;
  if (j >= qrows || nsplit <= 1) return;  // block-uniform
  const int d = f * 4;
  const int64_t ml_base = (int64_t)r * c.row_records + (int64_t)h * nsplit * qrows + j;
  const int64_t ml_step = qrows;
  const int g = j % c.G, i = j / c.G;
  fold_and_write<FC, SG>(red, c.part_o, c.part_ml, ml_base * c.D + d, ml_step * c.D, ml_base, ml_step, nsplit,
                         d < c.D, sg, f, c.out + r * c.o_sb + (int64_t)(h * c.G + g) * c.o_sh + (int64_t)i * c.o_st + d);
}

template <int DP>
static hipError_t launch_merge_capture_d(const CaptureArgs &c, int max_splits, hipStream_t stream) {
  constexpr int FC = DP / 4;
  const dim3 grid(c.total_items);
  if (max_splits <= 16 * (256 / FC))
    hipLaunchKernelGGL((merge_capture_kernel<DP, 256 / FC, 256>), grid, dim3(256), 0, stream, c);
  else if (max_splits <= 16 * (512 / FC))
    hipLaunchKernelGGL((merge_capture_kernel<DP, 512 / FC, 512>), grid, dim3(512), 0, stream, c);
  else
    hipLaunchKernelGGL((merge_capture_kernel<DP, 1024 / FC, 1024>), grid, dim3(1024), 0, stream, c);
  return hipGetLastError();
}

hipError_t launch_merge_capture(const CaptureArgs &c, int dp, int max_splits, hipStream_t stream) {
  switch (dp) {
    case 64: return launch_merge_capture_d<64>(c, max_splits, stream);
    case 128: return launch_merge_capture_d<128>(c, max_splits, stream);
    default: return launch_merge_capture_d<256>(c, max_splits, stream);
  }
}

hipError_t launch_merge(const MergeArgs &a, int dp, int max_splits, hipStream_t stream) {
  switch (dp) {
    case 64: return launch_merge_d<64, false>(a, nullptr, max_splits, a.total_items, stream);
    case 128: return launch_merge_d<128, false>(a, nullptr, max_splits, a.total_items, stream);
    default: return launch_merge_d<256, false>(a, nullptr, max_splits, a.total_items, stream);
  }
}

hipError_t launch_merge_dev(const MergeArgs *a, int dp, int max_splits, int64_t max_vectors, hipStream_t stream) {
  const MergeArgs none{};
  switch (dp) {
    case 64: return launch_merge_d<64, true>(none, a, max_splits, max_vectors, stream);
    case 128: return launch_merge_d<128, true>(none, a, max_splits, max_vectors, stream);
    default: return launch_merge_d<256, true>(none, a, max_splits, max_vectors, stream);
  }
}

}  // namespace xattn
