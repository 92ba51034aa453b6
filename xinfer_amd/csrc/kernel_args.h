// Kernel argument blocks shared by the host planner (capi.cpp) and the HIP
// kernels.  Plain structs passed by value through the kernarg segment; the
// per-row schedule travels inside them, so a launch needs no device metadata
// and no host<->device copy.
#pragma once

#include <stdint.h>

namespace xattn {

// Rows per launch.  Callers with more rows are split into several launches.
constexpr int kMaxRows = 64;

// One batch row as seen by a kernel.
struct RowSched {
  int32_t batch;        // index into the batch dimension
  int32_t count;        // real queries of this row (<= T); 0 = only zero its output
  int32_t length;       // populated KV length after the append (>= count, >= 1)
  int32_t item_begin;   // first work item (blockIdx.x) of this row
  int32_t nsplit;       // KV splits per group; 1 = no partial records
  int32_t ntiles;       // query tiles per kv head (prefill); 1 for decode
  int64_t rec_begin;    // first partial record of this row in the workspace
};
// Strided bf16 rank-4 tensor: element pointer + strides of dims 0..2 (dim 3 is unit).
struct View {
  const uint16_t *p;
  int64_t sb, sh, st;
};

struct AttnArgs {
  View q, k, v;
  uint16_t *out;             // [B, Hq, T, D]: unit feature stride, other strides multiples of 8
  int64_t o_sb, o_sh, o_st;  // contiguous: Hq*T*D, T*D, D; [B, T, Hq, D] storage: T*Hq*D, D, Hq*D
  float *part_o;             // [records][D] unnormalised fp32 partial outputs
  float *part_ml;            // [records][2] (running max in log2 units, sum)
  float scale_log2;          // softmax scale * log2(e)
  int32_t D, G, Hkv, T;
  int32_t total_items;       // work items of this launch (the decode grid may be smaller)
  int32_t nrows;
  RowSched rows[kMaxRows];
  // Prefill: items [xcd_begin[x], xcd_begin[x + 1]) run on XCD x (block b
  // runs item xcd_begin[b % 8] + b / 8 while below xcd_begin[b % 8 + 1]).
  // The planner cuts the item list into 8 runs of about equal work.
  int32_t xcd_begin[9];
  // Decode in-launch merge (decode.hip: merge_in_launch); null: split records
  // go to the merge launch.  One 64-bit arrival counter per decode item, the
  // one of a (row, kv head)'s first item serving it; every counter is left at
  // zero when the launch ends.  tag: nonzero, below 2^36, new for every
  // launch the host makes.
  uint64_t *arrive_ctr;
  uint64_t tag;
  // Page table (device, nullable): row r's K/V are k/v[page(r)], page(r) =
  // blocks[r * blocks_stride] clamped into [0, kv_rows); null: k/v[r].
  const int32_t *blocks;
  int64_t blocks_stride;
  int32_t kv_rows;  // size of k/v's batch dimension
};

// Merge of split partial records (merge.hip): one work item per query vector.
struct MergeRow {
  int32_t batch;
  int32_t count;       // real queries of the row
  int32_t nsplit;      // records per query vector (> 1)
  int32_t item_begin;  // first merge work item (blockIdx.x) of this row
  int32_t tiles;       // 0: [kv head][split][vector] records (decode); else the
                       // prefill layout: per (kv head, split, query tile of 128
                       // vectors) a block [D/4][128][4], `tiles` tiles per head
  int64_t rec_begin;   // first partial record of the row
};

struct MergeArgs {
  uint16_t *out;
  int64_t o_sb, o_sh, o_st;
  const float *part_o;
  const float *part_ml;
  int32_t D, G;
  int32_t total_items;  // query vectors to merge
  int32_t nrows;
  MergeRow rows[kMaxRows];
};

// Graph-capture decode (decode.hip, merge.hip): one launch shape serves every
// step, because the kernels read each row's query count and KV length from
// the device copy of the cumulative offsets instead of a host schedule.
// Records are laid out per row at capacity: row r's start at r * row_records,
// in the decode layout [kv head][split][vector] with the row's actual split
// count.  Counts are clamped to [0, min(T, C)] and lengths to [max(count, 1), C], so
// no device data can address outside q, k, v, out or the workspace.
struct CaptureArgs {
  View q, k, v;
  uint16_t *out;             // contiguous [B, Hq, T, D]
  int64_t o_sb, o_sh, o_st;
  float *part_o, *part_ml;   // records of every row at capacity
  const int32_t *offsets;    // device [2][B + 1]: cumulative counts, cumulative lengths
  float scale_log2;
  int32_t D, G, Hkv, T, B, C;
  int32_t tok_item;          // keys per decode work item
  int32_t total_items;       // decode: items at capacity; merge: query vectors at capacity
  int64_t row_records;       // records per row at capacity: Hkv * ceil(C / tok_item) * T * G
  const int32_t *blocks;     // page table as in AttnArgs (nullable), over the B rows of k/v
  int64_t blocks_stride;
};

// Graph-capture prefill: the arguments of a prefill launch and of its merge,
// planned on the device (prefill.hip: prefill_capture_plan_kernel) from the
// row counts and lengths in c.offsets, into *attn and *merge, which the
// prefill and merge kernels of the same graph then read.  Every row goes to
// the prefill kernel.  The limits are those the host sized the grids and the
// records for; the costs are the host planner's model (capi.cpp).
struct PrefillPlanArgs {
  CaptureArgs c;
  AttnArgs *attn;
  MergeArgs *merge;
  int32_t items_max;       // work items the records hold; the plan never exceeds it
  int32_t run_max;         // blocks per XCD of the prefill grid (8 * run_max blocks)
  int32_t splits_max;      // key splits a row may take (<= kMergeSerialSplits)
  int32_t min_split_keys;  // smallest split
  float tile_us;           // one 64-key tile of one item
  float item_us;           // fixed cost of an item
  float merge_us;          // the merge launch, when any row splits
  float record_us;         // one record (one query vector of one split) written and read
};

struct AppendArgs {
  View key, value;
  int64_t key_sd, value_sd;  // feature strides (1 on the vector path)
  const int64_t *positions;
  int64_t pos_sb, pos_st;
  const int32_t *cu_query;
  uint16_t *cache_key, *cache_value;  // contiguous [B, H, C, D]
  int32_t B, H, T, D, C;
};

// Query/key RMSNorm + rotary embedding + KV append (norm_rope.hip).
struct NormRopeArgs {
  View q, k, v;                        // [B, H, T, D] views of the projections
  const uint16_t *q_weight, *k_weight;  // [D] RMSNorm weights
  View cos, sin;                       // [B, T, D] (sb, st; sh unused)
  const int64_t *positions;
  int64_t pos_sb, pos_st;
  const int32_t *cu_query;
  uint16_t *q_out;                     // contiguous [B, Hq, T, D]
  uint16_t *cache_key, *cache_value;   // contiguous [B, Hkv, C, D]
  float eps;
  int32_t B, T, Hq, Hkv, D, C;
};

// Singleton projection (gemv.hip).
struct GemvArgs {
  const void *x;       // [k]
  const void *weight;  // [n, k] row-major
  void *out;           // [n]
  int64_t n, k;
};

}  // namespace xattn
