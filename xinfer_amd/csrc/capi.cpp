// C ABI of libxinfer_attention_ops.so: validation, work planning and launches.
//
// The planner turns host-side lengths into a static schedule carried in the
// kernel arguments (kernel_args.h): rows with at most 8 query vectors per KV
// head go to the split-KV decode kernel, the others to the MFMA prefill
// kernel; rows whose keys are split get fp32 partial records in the caller's
// workspace, combined by a merge launch after the attention kernels or, for
// small decode launches, by the last split of each (row, kv head) inside the
// decode launch (decode.hip: merge_in_launch), which folds in the merge
// launch's order and arithmetic.  The schedule is a function of the shapes and
// lengths only, never of tensor data, so results are deterministic and each
// row is isolated from the others' contents.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <functional>
#include <mutex>
#include <vector>

#include "xinfer_attention.h"
#include "kernel_args.h"
#include "launch.h"

namespace xattn {
namespace {

constexpr int kDecodeMaxQueryVectors = 8;  // G * count at or below this: decode kernel
constexpr int64_t kDecodeManyItems = 1536;  // one-round decode items from which items take several rounds
constexpr int kPrefillTileQ = 128;         // query vectors per prefill work item
constexpr int64_t kPrefillMinSplitKeys = 512;

int padded_dim(int64_t d) { return d <= 64 ? 64 : (d <= 128 ? 128 : 256); }
int pow2_at_least(int x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}
int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct Geometry {
  int64_t B, Hq, Hkv, T, D, C;
};

bool attention_layout_ok(const xinfer_view4 &t) {
  if (t.data == nullptr || (reinterpret_cast<uintptr_t>(t.data) & 15u) != 0) return false;
  if (t.size[3] > 1 && t.stride[3] != 1) return false;
  for (int i = 0; i < 3; ++i)
    if (t.size[i] > 1 && (t.stride[i] % 8) != 0) return false;
  // One (row, head) slice is addressed with 32-bit byte offsets.
  if ((t.size[2] + 1) * t.stride[2] * 2 >= (int64_t(1) << 31)) return false;
  return true;
}

// The prefill kernel addresses one batch row of Q ([Hq, T, D]) with 32-bit
// byte offsets from the row's first head.
bool query_layout_ok(const xinfer_view4 &q) {
  return (q.size[1] * q.stride[1] + q.size[2] * q.stride[2]) * 2 < (int64_t(1) << 31);
}

View view_of(const xinfer_view4 &t) {
  return View{static_cast<const uint16_t *>(t.data), t.stride[0], t.stride[1], t.stride[2]};
}

int check_heads_and_dim(const Geometry &g) {
  if (g.Hq <= 0 || g.Hkv <= 0 || g.Hq % g.Hkv != 0) return XINFER_ERR_HEADS;
  if (g.D < 8 || g.D > 256 || g.D % 8 != 0) return XINFER_ERR_HEAD_DIM;
  return XINFER_OK;
}

struct Group {
  int row0 = 0, nrows = 0;
  AttnArgs dec{};
  int dec_items = 0, dec_qr = 1, dec_rounds = 1;
  AttnArgs pre{};
  int pre_items = 0;
  MergeArgs merge{};
  int merge_items = 0, merge_max_splits = 0;
  // The decode launch may merge its split rows itself (decode_merge_fusable).
  bool dec_fusable = false;
};

struct Plan {
  std::vector<Group> groups;
  int64_t records = 0;
  int64_t D = 0;
  // Arrival counters of the decode in-launch merge: one per decode item of
  // the largest fusable group (the groups' launches run one after another and
  // leave every counter at zero).
  int64_t counters = 0;
  size_t part_ml_offset() const { return (size_t)((records * D * 4 + 255) / 256 * 256); }
  size_t counters_offset() const { return (part_ml_offset() + (size_t)records * 8 + 255) / 256 * 256; }
  size_t bytes() const { return records ? counters_offset() + (size_t)counters * 8 : 0; }
};

// Measured prefill costs on one MI355X CU, for the planner's choice of split
// size: one 64-key tile of a 128-vector item (D <= 128: 8 waves, two per
// SIMD; D = 256: 4 waves), and an item's fixed prologue, fold and epilogue.
double prefill_tile_us(int dp) { return dp <= 64 ? 0.9 : (dp <= 128 ? 1.15 : 1.9); }
constexpr double kPrefillItemUs = 4.5;
// Merge launch: fixed cost, and the record read at about 5 TB/s.
constexpr double kMergeLaunchUs = 5.0;
constexpr double kRecordBytesPerUs = 5.0e6;
constexpr int kCusPerXcd = 32;

// Decode merge choice.  The merge launch after a decode kernel costs an
// empty kernel's time there (1.8-2.1 us measured on MI355X) plus the cold
// round trip of its records (2-2.5 us).  The in-launch merge makes every
// block wait, before it retires, for its record stores and one counter round
// trip (kArrivalUs), which delays the blocks queued behind it once per wave of
// resident blocks, and leaves the last split of each (row, kv head) a fold at
// the tail (kInLaunchFoldUs).  Resident decode blocks: 256 CUs x 4 (the
// kernels take 96-220 VGPRs per lane).
constexpr double kDecodeMergeLaunchUs = 4.0;
constexpr double kArrivalUs = 1.5;
constexpr double kInLaunchFoldUs = 1.0;
constexpr int64_t kDecodeResidentBlocks = 1024;
// Decode kernel latency model: a launch floor, then whichever is longer of
// streaming the KV bytes and the rounds of the items each resident block
// runs one after another.
constexpr double kDecodeFloorUs = 2.0;
constexpr double kDecodeBytesPerUs = 5.5e6;
constexpr double kDecodeRoundUs = 1.2;

// Modelled time of a decode launch and its merge: `items` blocks of `rounds`
// rounds over kv_bytes; split: some row has several splits, merged in the
// launch (in_launch) or by the merge launch.
double decode_launch_us(int64_t items, int rounds, double kv_bytes, bool split, bool in_launch) {
  const double waves = (double)ceil_div(items, kDecodeResidentBlocks);
  double us = kDecodeFloorUs + std::max(kv_bytes / kDecodeBytesPerUs, rounds * kDecodeRoundUs * waves);
  if (split) us += in_launch ? kArrivalUs * waves + kInLaunchFoldUs : kDecodeMergeLaunchUs;
  return us;
}

// The in-launch merge pays when its block waits and tail fold cost less
// than the merge launch.
bool decode_merge_in_launch_pays(int64_t items) {
  return kArrivalUs * (double)ceil_div(items, kDecodeResidentBlocks) + kInLaunchFoldUs < kDecodeMergeLaunchUs;
}

// Rounds per decode item of rows [row0, row0 + nrows) (1 or
// kDecodeItemRounds).  Launches with at least kDecodeManyItems one-round
// items take kDecodeItemRounds: fewer, longer items cut the split records and
// per-item work.  Smaller launches compare, by decode_launch_us, one-round
// items against kDecodeItemRounds-round items when those bring every split
// row within the in-launch merge (fusable: Hkv a multiple of 8 and no split
// prefill row in the launch); longer items trade latency for the merge launch.
// Measured on MI355X (cfg3 seeds 1 and 3, one round + merge launch against
// four rounds + in-launch merge): 10.2 / 11.9 us and 13.6 / 12.8 us; the
// model picks the faster of each.
int choose_decode_rounds(const Geometry &g, const std::vector<int32_t> &counts, const std::vector<int32_t> &lengths,
                         int64_t row0, int nrows, int G, int dp, int qr, bool fusable) {
  int64_t items[2] = {0, 0}, max_splits[2] = {1, 1};
  double kv_bytes = 0;
  const int rounds[2] = {1, kDecodeItemRounds};
  for (int r = 0; r < nrows; ++r) {
    const int64_t qv = (int64_t)counts[row0 + r] * G, len = lengths[row0 + r];
    if (qv <= 0 || qv > kDecodeMaxQueryVectors) continue;
    kv_bytes += 4.0 * (double)(len * g.Hkv * g.D);
    for (int o = 0; o < 2; ++o) {
      const int64_t splits = ceil_div(len, rounds[o] * decode_tokens_per_item(dp, qr));
      items[o] += g.Hkv * splits;
      max_splits[o] = std::max(max_splits[o], splits);
    }
  }
  if (items[0] >= kDecodeManyItems) return kDecodeItemRounds;
  if (!fusable || max_splits[1] > kMergeSerialSplits) return 1;
  double us[2];
  for (int o = 0; o < 2; ++o) {
    const bool split = max_splits[o] > 1;
    const bool in_launch = max_splits[o] <= kMergeSerialSplits && decode_merge_in_launch_pays(items[o]);
    us[o] = decode_launch_us(items[o], rounds[o], kv_bytes, split, in_launch);
  }
  return us[1] < us[0] ? kDecodeItemRounds : 1;
}

// 64-key tiles of prefill item (split, query tile) of row rs: the key range
// of prefill.hip's split_range for that tile.
int64_t prefill_item_tiles(const RowSched &rs, int G, int split, int tile) {
  const int64_t qrows = (int64_t)rs.count * G, p0 = rs.length - rs.count;
  const int64_t j_last = std::min<int64_t>((int64_t)(tile + 1) * kPrefillTileQ, qrows) - 1;
  const int64_t kend = p0 + j_last / G + 1;
  const int64_t per = ceil_div(ceil_div(kend, rs.nsplit), 64) * 64;
  const int64_t ks0 = std::min(kend, split * per), ks1 = std::min(kend, ks0 + per);
  return ceil_div(ks1 - ks0, 64);
}

// Work of every prefill item of rows[0, nrows), in item order (row, kv head,
// split, query tile), in microseconds.
std::vector<double> prefill_item_work(const RowSched *rows, int nrows, int64_t Hkv, int G, int dp) {
  std::vector<double> work;
  for (int r = 0; r < nrows; ++r) {
    const RowSched &rs = rows[r];
    for (int64_t h = 0; h < Hkv; ++h)
      for (int split = 0; split < rs.nsplit; ++split)
        for (int tile = 0; tile < rs.ntiles; ++tile)
          work.push_back(prefill_item_tiles(rs, G, split, tile) * prefill_tile_us(dp) + kPrefillItemUs);
  }
  return work;
}

// Cut items (in order) into 8 contiguous runs of about equal work, one per
// XCD: on a ragged batch an equal number of items per XCD can leave the XCDs
// that hold the long rows with most of the work.  begin[0..8].
void xcd_runs(const std::vector<double> &work, int32_t *begin) {
  double total = 0;
  for (double w : work) total += w;
  begin[0] = 0;
  size_t i = 0;
  double done = 0;  // work of items [0, i)
  for (int x = 1; x < 8; ++x) {
    const double target = total * x / 8;
    // Take item i while that lands closer to the target than stopping before it.
    while (i < work.size() && (done + work[i]) - target < target - done) done += work[i++];
    begin[x] = (int32_t)i;
  }
  begin[8] = (int32_t)work.size();
}

// Time of the prefill launch when the items run as the hardware dispatches
// them: the blocks of each XCD, in order, to whichever of its CUs is free.
// The CUs' finishing times are kept in a min-heap (which of several tied CUs
// takes an item does not change the times that follow).
double simulated_prefill_us(const std::vector<double> &work) {
  int32_t begin[9];
  xcd_runs(work, begin);
  double span = 0;
  for (int x = 0; x < 8; ++x) {
    double free_at[kCusPerXcd] = {};  // all equal: already a heap
    for (int32_t i = begin[x]; i < begin[x + 1]; ++i) {
      std::pop_heap(free_at, free_at + kCusPerXcd, std::greater<double>());
      free_at[kCusPerXcd - 1] += work[(size_t)i];
      std::push_heap(free_at, free_at + kCusPerXcd, std::greater<double>());
    }
    span = std::max(span, *std::max_element(free_at, free_at + kCusPerXcd));
  }
  return span;
}

// Split count of a prefill row for keys-per-split `split_keys`.
int32_t prefill_splits(int64_t len, int64_t split_keys) {
  return (int32_t)std::max<int64_t>(1, ceil_div(len, split_keys));
}

// Keys per prefill split for the call: the split size, from about 256 to
// 2048 items' worth (at least kPrefillMinSplitKeys keys), whose launch,
// simulated as dispatched, plus its merge launch and the records' two trips
// through HBM, is fastest.  More, smaller items even out ragged rows; they
// cost per-item overhead, records and merge traffic.  The simulated span
// moves in jumps, when some row's split count changes, so the candidates are
// those change points: for each row and split count n, the smallest multiple
// of 64 keys that cuts the row into n splits (on the ragged D = 256 batch of
// 2235 tokens, cfg5, 3200-key splits measured 10 us faster than 2752-key
// ones, and 3264-key splits, one split fewer on one row, 4 us slower than
// 3200).  Candidates are simulated in increasing order of a lower bound on
// their time (total work over 256 CUs, or the longest item, plus the
// records), until that bound passes the best time found.
int64_t choose_split_keys(const Geometry &g, const std::vector<int32_t> &counts,
                          const std::vector<int32_t> &lengths, int G, int dp) {
  int64_t prefill_keys = 0;
  std::vector<RowSched> rows;
  for (int64_t r = 0; r < g.B; ++r) {
    const int64_t qv = (int64_t)counts[r] * G;
    if (qv <= kDecodeMaxQueryVectors) continue;
    prefill_keys += g.Hkv * ceil_div(qv, kPrefillTileQ) * lengths[r];
    RowSched rs{};
    rs.count = counts[r];
    rs.length = lengths[r];
    rs.ntiles = (int32_t)ceil_div(qv, kPrefillTileQ);
    rows.push_back(rs);
  }
  if (rows.empty()) return kPrefillMinSplitKeys;
  auto keys_for = [&](int64_t target) {
    return std::max(kPrefillMinSplitKeys, ceil_div(ceil_div(prefill_keys, target), 64) * 64);
  };
  const int64_t lo = keys_for(2048), hi = keys_for(256);
  std::vector<int64_t> keys = {lo, hi};
  for (const RowSched &rs : rows)
    for (int64_t n = ceil_div(rs.length, hi); n <= ceil_div(rs.length, lo); ++n) {
      const int64_t k = std::max(kPrefillMinSplitKeys, ceil_div(ceil_div(rs.length, n), 64) * 64);
      if (k >= lo && k <= hi) keys.push_back(k);
    }
  std::sort(keys.begin(), keys.end());
  keys.erase(std::unique(keys.begin(), keys.end()), keys.end());
  // Per row and split count: the work of one kv head's items and its longest
  // item (every kv head has the same items).
  struct RowWork {
    int32_t nsplit;
    double total, longest;
    std::vector<double> items;  // one kv head's items, in order (split, tile)
  };
  std::vector<std::vector<RowWork>> row_work(rows.size());
  auto work_of = [&](size_t r, int32_t nsplit) -> const RowWork & {
    for (const RowWork &w : row_work[r])
      if (w.nsplit == nsplit) return w;
    RowSched rs = rows[r];
    rs.nsplit = nsplit;
    RowWork w{nsplit, 0.0, 0.0, {}};
    w.items.reserve((size_t)nsplit * rs.ntiles);
    for (int split = 0; split < nsplit; ++split)
      for (int tile = 0; tile < rs.ntiles; ++tile) {
        const double us = prefill_item_tiles(rs, G, split, tile) * prefill_tile_us(dp) + kPrefillItemUs;
        w.total += us;
        w.longest = std::max(w.longest, us);
        w.items.push_back(us);
      }
    row_work[r].push_back(w);
    return row_work[r].back();
  };
  struct Candidate {
    double bound, records_us;
    int64_t split_keys;
  };
  std::vector<Candidate> cands;
  cands.reserve(keys.size());
  for (const int64_t split_keys : keys) {
    int64_t records = 0;
    double total = 0, longest = 0;
    for (size_t r = 0; r < rows.size(); ++r) {
      const int32_t nsplit = prefill_splits(rows[r].length, split_keys);
      if (nsplit > 1) records += g.Hkv * nsplit * rows[r].ntiles * kPrefillTileQ;
      const RowWork &w = work_of(r, nsplit);
      total += g.Hkv * w.total;
      longest = std::max(longest, w.longest);
    }
    // Records cross HBM twice: written by the prefill kernel, read by the merge.
    const double records_us =
        records ? kMergeLaunchUs + 2.0 * (double)records * (dp * 4 + 8) / kRecordBytesPerUs : 0.0;
    cands.push_back({std::max(total / (8.0 * kCusPerXcd), longest) + records_us, records_us, split_keys});
  }
  // Ties go to the larger split (fewer items and records).
  std::sort(cands.begin(), cands.end(), [](const Candidate &a, const Candidate &b) {
    return a.bound != b.bound ? a.bound < b.bound : a.split_keys > b.split_keys;
  });
  int64_t best_keys = cands.front().split_keys;
  double best_us = -1;
  std::vector<double> work;
  for (const Candidate &c : cands) {
    if (best_us >= 0 && c.bound >= best_us) break;
    // Items in launch order (row, kv head, split, tile), as prefill_item_work lists them.
    work.clear();
    for (size_t r = 0; r < rows.size(); ++r) {
      const RowWork &w = work_of(r, prefill_splits(rows[r].length, c.split_keys));
      for (int64_t h = 0; h < g.Hkv; ++h) work.insert(work.end(), w.items.begin(), w.items.end());
    }
    const double us = simulated_prefill_us(work) + c.records_us;
    if (best_us < 0 || us < best_us || (us == best_us && c.split_keys > best_keys)) {
      best_us = us;
      best_keys = c.split_keys;
    }
  }
  return best_keys;
}

// Whether a group's decode launch can merge its own split rows: it has split
// decode rows and no split prefill row (whose records need the merge launch
// anyway), every split row has at most kMergeSerialSplits splits (the merge
// layout the in-launch fold reproduces), and Hkv is a multiple of 8 (the
// kernel gives XCD x the kv heads h = x mod 8 of every row).
bool decode_merge_fusable(const Group &grp, int64_t Hkv) {
  if (grp.dec_items == 0 || grp.merge_items == 0 || Hkv % 8 != 0) return false;
  if (grp.merge_max_splits > kMergeSerialSplits) return false;
  for (int r = 0; r < grp.pre.nrows; ++r)
    if (grp.pre.rows[r].nsplit > 1) return false;
  return true;
}

// Whether this device deals consecutive blocks to its 8 XCDs in turn, probed
// once per device.  The probe runs on a private non-blocking stream, with
// this thread in relaxed capture mode, so that neither the caller's stream
// nor a capture another stream holds sees its launch, copy or synchronise.
// A first call made while the caller's stream is being captured skips the
// probe; until the probe has run, and if it disagrees, the merge launch is
// used.
bool xcd_dispatch_round_robin(hipStream_t stream) {
  constexpr int kMaxDevices = 64;
  static std::mutex lock;
  static int8_t known[kMaxDevices] = {};  // 0 unknown, 1 round robin, -1 not
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) return false;
  std::lock_guard<std::mutex> guard(lock);
  if (known[device] == 0) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &status) != hipSuccess || status != hipStreamCaptureStatusNone) return false;
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    if (hipThreadExchangeStreamCaptureMode(&mode) != hipSuccess) return false;
    hipStream_t probe_stream = nullptr;
    bool round_robin = false;
    hipError_t err = hipStreamCreateWithFlags(&probe_stream, hipStreamNonBlocking);
    if (err == hipSuccess) err = probe_xcd_dispatch(&round_robin, probe_stream);
    if (probe_stream != nullptr) (void)hipStreamDestroy(probe_stream);
    (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (err != hipSuccess) return false;
    known[device] = round_robin ? 1 : -1;
  }
  return known[device] == 1;
}

// XINFER_DECODE_MERGE_LAUNCH=1 keeps every decode split on the merge launch
// (read once per process): the check that both paths give the same bits.
bool merge_launch_forced() {
  static const bool forced = [] {
    const char *value = std::getenv("XINFER_DECODE_MERGE_LAUNCH");
    return value != nullptr && value[0] == '1';
  }();
  return forced;
}

// A nonzero tag below 2^36 for every decode launch with the in-launch merge.
uint64_t next_launch_tag() {
  static std::atomic<uint64_t> sequence{0};
  return sequence.fetch_add(1, std::memory_order_relaxed) % ((uint64_t(1) << 36) - 1) + 1;
}

// counts/lengths: per-row real queries and populated KV lengths (validated).
Plan make_plan(const Geometry &g, const std::vector<int32_t> &counts, const std::vector<int32_t> &lengths) {
  Plan plan;
  plan.D = g.D;
  const int G = (int)(g.Hq / g.Hkv);
  const int dp = padded_dim(g.D);

  // Keys per prefill split, chosen from the whole call's prefill work.
  const int64_t split_keys = choose_split_keys(g, counts, lengths, G, dp);

  for (int64_t row0 = 0; row0 < g.B; row0 += kMaxRows) {
    Group grp;
    grp.row0 = (int)row0;
    grp.nrows = (int)std::min<int64_t>(kMaxRows, g.B - row0);
    int max_qv = 1;
    for (int r = 0; r < grp.nrows; ++r) {
      const int qv = counts[row0 + r] * G;
      if (qv > 0 && qv <= kDecodeMaxQueryVectors) max_qv = std::max(max_qv, qv);
    }
    grp.dec_qr = pow2_at_least(max_qv);
    bool prefill_split = false;
    for (int r = 0; r < grp.nrows; ++r) {
      const int64_t qv = (int64_t)counts[row0 + r] * G;
      if (qv > kDecodeMaxQueryVectors && prefill_splits(lengths[row0 + r], split_keys) > 1) prefill_split = true;
    }
    grp.dec_rounds = choose_decode_rounds(g, counts, lengths, row0, grp.nrows, G, dp, grp.dec_qr,
                                          g.Hkv % 8 == 0 && !prefill_split);
    const int tpi = grp.dec_rounds * decode_tokens_per_item(dp, grp.dec_qr);
    for (int r = 0; r < grp.nrows; ++r) {
      const int64_t b = row0 + r;
      const int cnt = counts[b], len = lengths[b];
      const int64_t qv = (int64_t)cnt * G;
      RowSched rs{};
      rs.batch = (int32_t)b;
      rs.count = cnt;
      rs.length = len;
      rs.ntiles = 1;
      rs.nsplit = 1;
      const bool decode = qv <= kDecodeMaxQueryVectors;  // includes rows with no query (zero fill only)
      if (decode) {
        if (cnt > 0) rs.nsplit = (int32_t)ceil_div(len, tpi);
        rs.item_begin = grp.dec_items;
        grp.dec_items += (int)(g.Hkv * rs.nsplit);
      } else {
        rs.ntiles = (int32_t)ceil_div(qv, kPrefillTileQ);
        rs.nsplit = prefill_splits(len, split_keys);
        rs.item_begin = grp.pre_items;
        grp.pre_items += (int)(g.Hkv * rs.ntiles * rs.nsplit);
      }
      if (rs.nsplit > 1) {
        // Decode: [kv head][split][vector] records.  Prefill: per (kv head,
        // split, query tile) a block of kPrefillTileQ records.
        rs.rec_begin = plan.records;
        plan.records += g.Hkv * rs.nsplit * (decode ? qv : rs.ntiles * kPrefillTileQ);
        MergeRow &mr = grp.merge.rows[grp.merge.nrows++];
        mr.batch = (int32_t)b;
        mr.count = cnt;
        mr.nsplit = rs.nsplit;
        mr.item_begin = grp.merge_items;
        mr.tiles = decode ? 0 : rs.ntiles;
        mr.rec_begin = rs.rec_begin;
        grp.merge_items += (int)(g.Hkv * qv);
        grp.merge_max_splits = std::max(grp.merge_max_splits, (int)rs.nsplit);
      }
      AttnArgs &a = decode ? grp.dec : grp.pre;
      a.rows[a.nrows++] = rs;
    }
    grp.dec_fusable = decode_merge_fusable(grp, g.Hkv);
    if (grp.dec_fusable) plan.counters = std::max<int64_t>(plan.counters, grp.dec_items);
    if (grp.pre_items > 0) xcd_runs(prefill_item_work(grp.pre.rows, grp.pre.nrows, g.Hkv, G, dp), grp.pre.xcd_begin);
    plan.groups.push_back(grp);
  }
  return plan;
}

// The plan of this thread's last call.  A model step calls the operator once
// per layer with the same counts and lengths, and every call plans twice (its
// workspace size, then the launch), while planning a ragged prefill batch
// simulates its dispatch at several split sizes (about 0.36 ms for the
// batch-8 D = 256 prefill of 2235 tokens); a call whose geometry, counts and
// lengths equal the last one's reuses that plan.  A plan depends on nothing
// else: not on the device, the stream or the tensors' addresses.
Plan cached_plan(const Geometry &g, const std::vector<int32_t> &counts, const std::vector<int32_t> &lengths) {
  struct Entry {
    bool valid = false;
    Geometry g{};
    std::vector<int32_t> counts, lengths;
    Plan plan;
  };
  thread_local Entry last;
  const bool same = last.valid && last.g.B == g.B && last.g.Hq == g.Hq && last.g.Hkv == g.Hkv &&
                    last.g.T == g.T && last.g.D == g.D && last.g.C == g.C && last.counts == counts &&
                    last.lengths == lengths;
  if (!same) {
    last.valid = false;
    last.plan = make_plan(g, counts, lengths);
    last.g = g;
    last.counts = counts;
    last.lengths = lengths;
    last.valid = true;
  }
  return last.plan;
}

// A page table (nullable) is a device int32 pointer with a non-negative row stride.
int check_blocks(const int32_t *blocks, int64_t blocks_stride) {
  if (blocks == nullptr) return XINFER_OK;
  if ((reinterpret_cast<uintptr_t>(blocks) & 3u) != 0 || blocks_stride < 0) return XINFER_ERR_ARGUMENT;
  return XINFER_OK;
}

int run_plan(const Plan &plan, const Geometry &g, const xinfer_view4 &q, const xinfer_view4 &k,
             const xinfer_view4 &v, const int32_t *blocks, int64_t blocks_stride, double scale,
             const xinfer_view4 &out, void *workspace, hipStream_t stream) {
  const int G = (int)(g.Hq / g.Hkv);
  const int dp = padded_dim(g.D);
  float *part_o = static_cast<float *>(workspace);
  float *part_ml =
      plan.records ? reinterpret_cast<float *>(static_cast<char *>(workspace) + plan.part_ml_offset())
                   : nullptr;
  for (Group grp : plan.groups) {
    for (AttnArgs *a : {&grp.dec, &grp.pre}) {
      a->q = view_of(q);
      a->k = view_of(k);
      a->v = view_of(v);
      a->out = static_cast<uint16_t *>(const_cast<void *>(out.data));
      a->o_sb = out.stride[0];
      a->o_sh = out.stride[1];
      a->o_st = out.stride[2];
      a->part_o = part_o;
      a->part_ml = part_ml;
      a->scale_log2 = (float)(scale * 1.4426950408889634);
      a->D = (int32_t)g.D;
      a->G = G;
      a->Hkv = (int32_t)g.Hkv;
      a->T = (int32_t)g.T;
      a->blocks = blocks;
      a->blocks_stride = blocks_stride;
      a->kv_rows = (int32_t)g.B;
    }
    grp.dec.total_items = grp.dec_items;
    grp.pre.total_items = grp.pre_items;
    grp.dec.arrive_ctr = nullptr;
    grp.dec.tag = 0;
    if (grp.dec_fusable && !merge_launch_forced() && decode_merge_in_launch_pays(grp.dec_items) &&
        xcd_dispatch_round_robin(stream)) {
      grp.dec.arrive_ctr = reinterpret_cast<uint64_t *>(static_cast<char *>(workspace) + plan.counters_offset());
      grp.dec.tag = next_launch_tag();
      grp.merge_items = 0;  // every split row is a decode row, merged in the launch
    }
    if (grp.dec_items > 0 && launch_decode(grp.dec, dp, grp.dec_qr, grp.dec_rounds, grp.dec_items, stream) != hipSuccess)
      return XINFER_ERR_LAUNCH;
    if (grp.pre_items > 0 && launch_prefill(grp.pre, dp, stream) != hipSuccess) return XINFER_ERR_LAUNCH;
    if (grp.merge_items > 0) {
      MergeArgs &m = grp.merge;
      m.out = static_cast<uint16_t *>(const_cast<void *>(out.data));
      m.o_sb = out.stride[0];
      m.o_sh = out.stride[1];
      m.o_st = out.stride[2];
      m.part_o = part_o;
      m.part_ml = part_ml;
      m.D = (int32_t)g.D;
      m.G = G;
      m.total_items = grp.merge_items;
      if (launch_merge(m, dp, grp.merge_max_splits, stream) != hipSuccess) return XINFER_ERR_LAUNCH;
    }
  }
  return XINFER_OK;
}

// The contiguous [B, Hq, T, D] output the operators allocate.
xinfer_view4 contiguous_output(const Geometry &g, void *out) {
  xinfer_view4 o{};
  o.data = out;
  const int64_t sizes[4] = {g.B, g.Hq, g.T, g.D};
  const int64_t strides[4] = {g.Hq * g.T * g.D, g.T * g.D, g.D, 1};
  for (int i = 0; i < 4; ++i) {
    o.size[i] = sizes[i];
    o.stride[i] = strides[i];
  }
  return o;
}

// An output view the kernels can write: q's sizes, unit feature stride, the
// other strides multiples of 8 elements, 16-byte aligned data.
int check_output(const Geometry &g, const xinfer_view4 *out) {
  if (out == nullptr || out->data == nullptr) return XINFER_ERR_ARGUMENT;
  const int64_t sizes[4] = {g.B, g.Hq, g.T, g.D};
  for (int i = 0; i < 4; ++i)
    if (out->size[i] != sizes[i]) return XINFER_ERR_QKV_SHAPES;
  if ((reinterpret_cast<uintptr_t>(out->data) & 15u) != 0 || out->stride[3] != 1) return XINFER_ERR_LAYOUT;
  for (int i = 0; i < 3; ++i)
    if (out->stride[i] % 8 != 0 || out->stride[i] < 0) return XINFER_ERR_LAYOUT;
  return XINFER_OK;
}

// Validation of xinfer::flash_attention (attention.cpp:84-104), in its order.
int check_flash(const xinfer_view4 *q, const xinfer_view4 *k, const xinfer_view4 *v,
                int64_t valid_length, Geometry &g) {
  if (!q || !k || !v) return XINFER_ERR_ARGUMENT;
  g = Geometry{q->size[0], q->size[1], k->size[1], q->size[2], q->size[3], k->size[2]};
  if (!(g.B > 0 && g.T >= 1 && g.T <= 512)) return XINFER_ERR_Q_SHAPE;
  bool same = true;
  for (int i = 0; i < 4; ++i) same = same && v->size[i] == k->size[i];
  if (!(k->size[0] == g.B && g.C > 0 && k->size[3] == g.D && same)) return XINFER_ERR_KV_SHAPE;
  if (int rc = check_heads_and_dim(g)) return rc;
  if (!(valid_length >= g.T && valid_length <= g.C)) return XINFER_ERR_PREFIX;
  return XINFER_OK;
}

// Validation of xinfer::batched_flash_attention (attention.cpp:17-45).
int check_batched(const xinfer_view4 *q, const xinfer_view4 *k, const xinfer_view4 *v,
                  const int32_t *offsets, Geometry &g, std::vector<int32_t> &counts,
                  std::vector<int32_t> &lengths) {
  if (!q || !k || !v || !offsets) return XINFER_ERR_ARGUMENT;
  g = Geometry{q->size[0], q->size[1], k->size[1], q->size[2], q->size[3], k->size[2]};
  bool same = true;
  for (int i = 0; i < 4; ++i) same = same && v->size[i] == k->size[i];
  if (!(same && k->size[0] == g.B && k->size[3] == g.D) || g.B < 0 || g.T < 0)
    return XINFER_ERR_QKV_SHAPES;
  if (int rc = check_heads_and_dim(g)) return rc;
  const int32_t *cuq = offsets, *cuk = offsets + g.B + 1;
  if (cuq[0] != 0 || cuk[0] != 0) return XINFER_ERR_OFFSETS_START;
  counts.resize(g.B);
  lengths.resize(g.B);
  for (int64_t r = 0; r < g.B; ++r) {
    const int64_t count = (int64_t)cuq[r + 1] - cuq[r], length = (int64_t)cuk[r + 1] - cuk[r];
    if (!(count >= 0 && count <= g.T && length >= count && length >= 1 && length <= g.C))
      return XINFER_ERR_LENGTHS;
    counts[r] = (int32_t)count;
    lengths[r] = (int32_t)length;
  }
  return XINFER_OK;
}

// Graph-capture mode (xinfer_batched_flash_attention_graph): a plan that
// depends only on the shapes.  Rows must take the decode kernel (at most
// kDecodeMaxQueryVectors query vectors per KV head, i.e. T * G <= 8) and fit
// one row table (B <= kMaxRows, which the kernels' per-block tables assume).
// Records are laid out for every row at capacity.
struct CapturePlan {
  int dp = 0, qr = 1, rounds = 1, tok_item = 0, splits_max = 0, decode_blocks = 0;
  int64_t row_records = 0, records = 0;
  int64_t dp_d = 0;  // the head dim D (records hold D floats)
  // Prefill shapes (T * Hq/Hkv > 8): every row takes the prefill kernel,
  // planned on the device; the workspace also holds the prefill and merge
  // arguments the plan kernel writes.
  bool prefill = false;
  int64_t items_max = 0, vectors_max = 0;
  size_t part_ml_offset() const { return (size_t)((records * dp_d * 4 + 255) / 256 * 256); }
  size_t records_bytes() const { return records ? part_ml_offset() + (size_t)records * 8 : 0; }
  size_t attn_offset() const { return (records_bytes() + 255) / 256 * 256; }
  size_t merge_offset() const { return attn_offset() + (sizeof(AttnArgs) + 255) / 256 * 256; }
  size_t bytes() const { return prefill ? merge_offset() + sizeof(MergeArgs) : records_bytes(); }
};
// Decode blocks of a capture launch: every item of the capacity layout, at
// most eight per CU of the 256.  With one-round items the blocks take the
// valid items in turn; multi-round items (kDecodeItemRounds rounds, chosen
// when the capacity layout has as many one-round items as the default
// planner's threshold and its multi-round items fit this grid) take one block
// each.
constexpr int kCaptureMaxBlocks = 2048;

int check_capture(const xinfer_view4 *q, const xinfer_view4 *k, const xinfer_view4 *v, Geometry &g,
                  CapturePlan &cp) {
  if (!q || !k || !v) return XINFER_ERR_ARGUMENT;
  g = Geometry{q->size[0], q->size[1], k->size[1], q->size[2], q->size[3], k->size[2]};
  bool same = true;
  for (int i = 0; i < 4; ++i) same = same && v->size[i] == k->size[i];
  if (!(same && k->size[0] == g.B && k->size[3] == g.D) || g.B < 0 || g.T < 0 || g.C <= 0)
    return XINFER_ERR_QKV_SHAPES;
  if (int rc = check_heads_and_dim(g)) return rc;
  const int64_t G = g.Hq / g.Hkv;
  if (g.B > kMaxRows) return XINFER_ERR_CAPTURE_ROWS;
  cp.dp = padded_dim(g.D);
  cp.dp_d = g.D;
  if (g.T * G > kDecodeMaxQueryVectors) {
    // Prefill shapes: the device plan (prefill.hip:
    // prefill_capture_plan_kernel) picks the split size from the lengths, in
    // the range choose_split_keys searches, so that the items stay below
    // 2048 + one per (row, kv head, query tile); no row takes more than
    // kMergeSerialSplits splits (or splits below kPrefillMinSplitKeys keys).
    // The prefill grid, the records and the merge grid are sized for that.
    cp.prefill = true;
    const int64_t unsplit = g.B * g.Hkv * ceil_div(g.T * G, kPrefillTileQ);
    cp.splits_max = (int)std::min<int64_t>(kMergeSerialSplits, ceil_div(g.C, kPrefillMinSplitKeys));
    cp.items_max = std::min(2048 + unsplit, unsplit * cp.splits_max);
    cp.vectors_max = g.B * g.Hkv * g.T * G;
    cp.records = cp.splits_max > 1 ? cp.items_max * kPrefillTileQ : 0;
    // Item, record and vector indices are 32-bit on the device (a q tensor
    // that large would not fit in memory).
    if (cp.items_max * kPrefillTileQ >= (int64_t(1) << 31) || cp.vectors_max >= (int64_t(1) << 31))
      return XINFER_ERR_QKV_SHAPES;
    return XINFER_OK;
  }
  cp.qr = pow2_at_least((int)std::max<int64_t>(1, g.T * G));
  const int tok_round = decode_tokens_per_item(cp.dp, cp.qr);
  const int64_t one_round_items = g.B * g.Hkv * ceil_div(g.C, tok_round);
  const int64_t multi_round_items = g.B * g.Hkv * ceil_div(g.C, (int64_t)kDecodeItemRounds * tok_round);
  cp.rounds = one_round_items >= kDecodeManyItems && multi_round_items <= kCaptureMaxBlocks ? kDecodeItemRounds : 1;
  cp.tok_item = cp.rounds * tok_round;
  cp.splits_max = (int)ceil_div(g.C, cp.tok_item);
  cp.row_records = g.Hkv * cp.splits_max * g.T * G;
  cp.records = cp.splits_max > 1 ? g.B * cp.row_records : 0;
  cp.decode_blocks = (int)std::min<int64_t>(std::max<int64_t>(1, g.B * g.Hkv * cp.splits_max), kCaptureMaxBlocks);
  return XINFER_OK;
}

// The caller's workspace: at least `need` bytes, 16-byte aligned (the records
// take 16-byte stores; the argument blocks planned on the device are read
// with scalar loads).  A workspace of zero bytes may be null.
int check_workspace(const void *workspace, size_t bytes, size_t need) {
  if (bytes < need || (need && workspace == nullptr) || (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0)
    return XINFER_ERR_WORKSPACE;
  return XINFER_OK;
}

int check_common(const xinfer_view4 &q, const xinfer_view4 &k, const xinfer_view4 &v, double scale) {
  if (!(std::isfinite(scale) && scale > 0)) return XINFER_ERR_SCALE;
  if (!attention_layout_ok(q) || !query_layout_ok(q) || !attention_layout_ok(k) ||
      !attention_layout_ok(v))
    return XINFER_ERR_LAYOUT;
  return XINFER_OK;
}

}  // namespace
}  // namespace xattn

using namespace xattn;

extern "C" {

const char *xinfer_status_string(int status) {
  switch (status) {
    case XINFER_OK: return "Success";
    case XINFER_ERR_QKV_SHAPES: return "Invalid Q/K/V shapes";
    case XINFER_ERR_Q_SHAPE: return "Unsupported Q shape";
    case XINFER_ERR_KV_SHAPE:
      return "Expected matching full-capacity K/V inputs [batch,kv_heads,capacity,head_dim]";
    case XINFER_ERR_HEADS: return "Query heads must be a positive multiple of KV heads";
    case XINFER_ERR_HEAD_DIM: return "Flash head dimension must be a multiple of 8 in 8..256";
    case XINFER_ERR_PREFIX: return "Invalid valid-prefix length";
    case XINFER_ERR_SCALE: return "Attention scale must be finite and positive";
    case XINFER_ERR_OFFSETS_START: return "Cumulative lengths must start at zero";
    case XINFER_ERR_LENGTHS: return "Invalid query/KV lengths";
    case XINFER_ERR_WORKSPACE: return "Attention workspace is smaller than its size query or not 16-byte aligned";
    case XINFER_ERR_LAYOUT:
      return "Attention tensors need a unit feature stride, strides divisible by 8 and 16-byte "
             "aligned data";
    case XINFER_ERR_CACHE:
      return "Expected contiguous KV caches [batch,kv_heads,capacity,head_dim] matching key/value";
    case XINFER_ERR_LAUNCH: return "HIP kernel launch failed";
    case XINFER_ERR_ARGUMENT: return "Invalid argument";
    case XINFER_ERR_ROPE_SHAPE:
      return "Expected q [B,Hq,T,D], key/value [B,Hkv,T,D] and cos/sin [B,1,T,D] with D in {64,128,256}";
    case XINFER_ERR_EPS: return "RMSNorm epsilon must be finite and non-negative";
    case XINFER_ERR_CAPTURE_ROWS:
      return "Graph-capture attention takes at most 64 rows";
    case XINFER_ERR_SCRATCH:
      return "Attention needs more split-record scratch than the allocation-free entry point holds (32 MiB)";
    default: return "Unknown xinfer status";
  }
}

size_t xinfer_batched_flash_attention_workspace_size(const xinfer_view4 *q, const xinfer_view4 *k,
                                                     const int32_t *host_offsets) {
  Geometry g;
  std::vector<int32_t> counts, lengths;
  if (check_batched(q, k, k, host_offsets, g, counts, lengths) != XINFER_OK) return 0;
  return cached_plan(g, counts, lengths).bytes();
}

int xinfer_batched_flash_attention(const xinfer_view4 *q, const xinfer_view4 *k,
                                   const xinfer_view4 *v, const int32_t *host_offsets,
                                   const int32_t *blocks, int64_t blocks_stride, double scale,
                                   void *out, void *workspace, size_t workspace_bytes,
                                   void *stream) {
  Geometry g;
  std::vector<int32_t> counts, lengths;
  if (int rc = check_batched(q, k, v, host_offsets, g, counts, lengths)) return rc;
  if (int rc = check_common(*q, *k, *v, scale)) return rc;
  if (int rc = check_blocks(blocks, blocks_stride)) return rc;
  if (g.B == 0 || g.T == 0) return XINFER_OK;
  if (out == nullptr) return XINFER_ERR_ARGUMENT;
  const Plan plan = cached_plan(g, counts, lengths);
  if (int rc = check_workspace(workspace, workspace_bytes, plan.bytes())) return rc;
  return run_plan(plan, g, *q, *k, *v, blocks, blocks_stride, scale, contiguous_output(g, out), workspace,
                  static_cast<hipStream_t>(stream));
}

size_t xinfer_batched_flash_attention_graph_workspace_size(const xinfer_view4 *q, const xinfer_view4 *k) {
  Geometry g;
  CapturePlan cp;
  if (check_capture(q, k, k, g, cp) != XINFER_OK) return 0;
  return cp.bytes();
}

int xinfer_batched_flash_attention_graph(const xinfer_view4 *q, const xinfer_view4 *k, const xinfer_view4 *v,
                                         const int32_t *device_offsets, const int32_t *blocks,
                                         int64_t blocks_stride, double scale, void *out, void *workspace,
                                         size_t workspace_bytes, void *stream) {
  Geometry g;
  CapturePlan cp;
  if (int rc = check_capture(q, k, v, g, cp)) return rc;
  if (int rc = check_common(*q, *k, *v, scale)) return rc;
  if (int rc = check_blocks(blocks, blocks_stride)) return rc;
  if (g.B == 0 || g.T == 0) return XINFER_OK;
  if (out == nullptr || device_offsets == nullptr) return XINFER_ERR_ARGUMENT;
  if (int rc = check_workspace(workspace, workspace_bytes, cp.bytes())) return rc;
  CaptureArgs c{};
  c.q = view_of(*q);
  c.k = view_of(*k);
  c.v = view_of(*v);
  c.out = static_cast<uint16_t *>(out);
  c.o_sb = g.Hq * g.T * g.D;
  c.o_sh = g.T * g.D;
  c.o_st = g.D;
  c.part_o = static_cast<float *>(workspace);
  c.part_ml = cp.records ? reinterpret_cast<float *>(static_cast<char *>(workspace) + cp.part_ml_offset()) : nullptr;
  c.offsets = device_offsets;
  c.scale_log2 = (float)(scale * 1.4426950408889634);
  c.D = (int32_t)g.D;
  c.G = (int32_t)(g.Hq / g.Hkv);
  c.Hkv = (int32_t)g.Hkv;
  c.T = (int32_t)g.T;
  c.B = (int32_t)g.B;
  c.C = (int32_t)g.C;
  c.tok_item = cp.tok_item;
  c.row_records = cp.row_records;
  c.blocks = blocks;
  c.blocks_stride = blocks_stride;
  c.total_items = (int32_t)(g.B * g.Hkv * cp.splits_max);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  if (cp.prefill) {
    char *ws = static_cast<char *>(workspace);
    PrefillPlanArgs pp{};
    pp.c = c;
    pp.attn = reinterpret_cast<AttnArgs *>(ws + cp.attn_offset());
    pp.merge = reinterpret_cast<MergeArgs *>(ws + cp.merge_offset());
    pp.items_max = (int32_t)cp.items_max;
    // 8 XCD runs of at most ceil(items_max / 8) items (the plan clamps its cuts).
    pp.run_max = (int32_t)ceil_div(cp.items_max, 8);
    pp.splits_max = cp.splits_max;
    pp.min_split_keys = (int32_t)kPrefillMinSplitKeys;
    pp.tile_us = (float)prefill_tile_us(cp.dp);
    pp.item_us = (float)kPrefillItemUs;
    pp.merge_us = (float)kMergeLaunchUs;
    pp.record_us = (float)(2.0 * (cp.dp * 4 + 8) / kRecordBytesPerUs);
    if (launch_prefill_capture(pp, cp.dp, (unsigned)(8 * pp.run_max), s) != hipSuccess) return XINFER_ERR_LAUNCH;
    if (cp.splits_max > 1 && launch_merge_dev(pp.merge, cp.dp, cp.splits_max, cp.vectors_max, s) != hipSuccess)
      return XINFER_ERR_LAUNCH;
    return XINFER_OK;
  }
  if (launch_decode_capture(c, cp.dp, cp.qr, cp.rounds, cp.decode_blocks, s) != hipSuccess) return XINFER_ERR_LAUNCH;
  if (cp.splits_max > 1) {
    c.total_items = (int32_t)(g.B * g.Hkv * g.T * c.G);
    if (launch_merge_capture(c, cp.dp, cp.splits_max, s) != hipSuccess) return XINFER_ERR_LAUNCH;
  }
  return XINFER_OK;
}

int xinfer_batched_flash_attention_noalloc(const xinfer_view4 *q, const xinfer_view4 *k,
                                           const xinfer_view4 *v, const int32_t *host_offsets,
                                           const int32_t *blocks, int64_t blocks_stride, double scale,
                                           void *out, void *stream) {
  static_assert(kScratchBytes == XINFER_NOALLOC_SCRATCH_BYTES, "scratch size of the C header");
  Geometry g;
  std::vector<int32_t> counts, lengths;
  if (int rc = check_batched(q, k, v, host_offsets, g, counts, lengths)) return rc;
  if (int rc = check_common(*q, *k, *v, scale)) return rc;
  if (int rc = check_blocks(blocks, blocks_stride)) return rc;
  if (g.B == 0 || g.T == 0) return XINFER_OK;
  if (out == nullptr) return XINFER_ERR_ARGUMENT;
  const Plan plan = cached_plan(g, counts, lengths);
  if (plan.bytes() > kScratchBytes) return XINFER_ERR_SCRATCH;
  // The device address of the static scratch on the current device (never
  // the host-side name of the array).
  void *records = nullptr;
  if (plan.bytes() > 0 && scratch_pointer(&records) != hipSuccess) return XINFER_ERR_LAUNCH;
  return run_plan(plan, g, *q, *k, *v, blocks, blocks_stride, scale, contiguous_output(g, out), records,
                  static_cast<hipStream_t>(stream));
}

int xinfer_batched_flash_attention_out(const xinfer_view4 *q, const xinfer_view4 *k, const xinfer_view4 *v,
                                       const int32_t *host_offsets, const int32_t *blocks,
                                       int64_t blocks_stride, double scale, const xinfer_view4 *out,
                                       void *workspace, size_t workspace_bytes, void *stream) {
  Geometry g;
  std::vector<int32_t> counts, lengths;
  if (int rc = check_batched(q, k, v, host_offsets, g, counts, lengths)) return rc;
  if (int rc = check_common(*q, *k, *v, scale)) return rc;
  if (int rc = check_blocks(blocks, blocks_stride)) return rc;
  if (g.B == 0 || g.T == 0) return XINFER_OK;
  if (int rc = check_output(g, out)) return rc;
  const Plan plan = cached_plan(g, counts, lengths);
  if (int rc = check_workspace(workspace, workspace_bytes, plan.bytes())) return rc;
  return run_plan(plan, g, *q, *k, *v, blocks, blocks_stride, scale, *out, workspace,
                  static_cast<hipStream_t>(stream));
}

size_t xinfer_flash_attention_workspace_size(const xinfer_view4 *q, const xinfer_view4 *k,
                                             int64_t valid_length) {
  Geometry g;
  if (check_flash(q, k, k, valid_length, g) != XINFER_OK) return 0;
  std::vector<int32_t> counts(g.B, (int32_t)g.T), lengths(g.B, (int32_t)valid_length);
  return cached_plan(g, counts, lengths).bytes();
}

int xinfer_flash_attention(const xinfer_view4 *q, const xinfer_view4 *k, const xinfer_view4 *v,
                           int64_t valid_length, double scale, void *out, void *workspace,
                           size_t workspace_bytes, void *stream) {
  Geometry g;
  if (int rc = check_flash(q, k, v, valid_length, g)) return rc;
  if (int rc = check_common(*q, *k, *v, scale)) return rc;
  if (out == nullptr) return XINFER_ERR_ARGUMENT;
  std::vector<int32_t> counts(g.B, (int32_t)g.T), lengths(g.B, (int32_t)valid_length);
  const Plan plan = cached_plan(g, counts, lengths);
  if (int rc = check_workspace(workspace, workspace_bytes, plan.bytes())) return rc;
  return run_plan(plan, g, *q, *k, *v, nullptr, 0, scale, contiguous_output(g, out), workspace,
                  static_cast<hipStream_t>(stream));
}

int xinfer_append_kv_batched(const xinfer_view4 *key, const xinfer_view4 *value,
                             const int64_t *positions, int64_t pos_stride_b, int64_t pos_stride_t,
                             const int32_t *cu_query, const xinfer_view4 *cache_key,
                             const xinfer_view4 *cache_value, void *stream) {
  if (!key || !value || !cache_key || !cache_value) return XINFER_ERR_ARGUMENT;
  const int64_t B = key->size[0], H = key->size[1], T = key->size[2], D = key->size[3];
  for (int i = 0; i < 4; ++i)
    if (value->size[i] != key->size[i] || key->size[i] < 0) return XINFER_ERR_ARGUMENT;
  if (B == 0 || H == 0 || T == 0 || D == 0) return XINFER_OK;
  if (!positions || !cu_query || !key->data || !value->data) return XINFER_ERR_ARGUMENT;
  for (const xinfer_view4 *c : {cache_key, cache_value}) {
    if (!c->data || c->size[0] < B || c->size[1] != H || c->size[3] != D || c->size[2] <= 0)
      return XINFER_ERR_CACHE;
    if (c->stride[3] != 1 || c->stride[2] != D || c->stride[1] != c->size[2] * D ||
        c->stride[0] != H * c->size[2] * D)
      return XINFER_ERR_CACHE;
    for (int i = 0; i < 4; ++i)
      if (c->size[i] != cache_key->size[i]) return XINFER_ERR_CACHE;
  }
  AppendArgs a{};
  a.key = view_of(*key);
  a.value = view_of(*value);
  a.key_sd = key->stride[3];
  a.value_sd = value->stride[3];
  a.positions = positions;
  a.pos_sb = pos_stride_b;
  a.pos_st = pos_stride_t;
  a.cu_query = cu_query;
  a.cache_key = static_cast<uint16_t *>(const_cast<void *>(cache_key->data));
  a.cache_value = static_cast<uint16_t *>(const_cast<void *>(cache_value->data));
  a.B = (int32_t)B;
  a.H = (int32_t)H;
  a.T = (int32_t)T;
  a.D = (int32_t)D;
  a.C = (int32_t)cache_key->size[2];
  auto vec_ok = [&](const xinfer_view4 &t) {
    if ((reinterpret_cast<uintptr_t>(t.data) & 15u) != 0 || t.stride[3] != 1 || D % 8 != 0) return false;
    for (int i = 0; i < 3; ++i)
      if (t.size[i] > 1 && t.stride[i] % 8 != 0) return false;
    return true;
  };
  const bool vector = vec_ok(*key) && vec_ok(*value) &&
                      (reinterpret_cast<uintptr_t>(cache_key->data) & 15u) == 0 &&
                      (reinterpret_cast<uintptr_t>(cache_value->data) & 15u) == 0;
  return launch_append(a, vector, static_cast<hipStream_t>(stream)) == hipSuccess ? XINFER_OK
                                                                                  : XINFER_ERR_LAUNCH;
}

int xinfer_qk_norm_rope_append(const xinfer_view4 *q, const xinfer_view4 *key, const xinfer_view4 *value,
                               const void *q_weight, const void *k_weight, double eps,
                               const xinfer_view4 *cos, const xinfer_view4 *sin, const int64_t *positions,
                               int64_t pos_stride_b, int64_t pos_stride_t, const int32_t *cu_query,
                               void *q_out, const xinfer_view4 *cache_key, const xinfer_view4 *cache_value,
                               void *stream) {
  if (!q || !key || !value || !cos || !sin || !cache_key || !cache_value) return XINFER_ERR_ARGUMENT;
  const int64_t B = q->size[0], Hq = q->size[1], T = q->size[2], D = q->size[3], Hkv = key->size[1];
  for (int i = 0; i < 4; ++i)
    if (q->size[i] < 0 || key->size[i] < 0 || value->size[i] != key->size[i]) return XINFER_ERR_ROPE_SHAPE;
  if (key->size[0] != B || key->size[2] != T || key->size[3] != D || Hq <= 0 || Hkv <= 0 ||
      (D != 64 && D != 128 && D != 256))
    return XINFER_ERR_ROPE_SHAPE;
  for (const xinfer_view4 *r : {cos, sin})
    if (r->size[0] != B || r->size[1] != 1 || r->size[2] != T || r->size[3] != D) return XINFER_ERR_ROPE_SHAPE;
  if (!(std::isfinite(eps) && eps >= 0)) return XINFER_ERR_EPS;
  if (B == 0 || T == 0) return XINFER_OK;
  if (!q_weight || !k_weight || !positions || !cu_query || !q_out) return XINFER_ERR_ARGUMENT;
  // 16-byte rows: unit feature stride, other strides divisible by 8, aligned data.
  auto rows_ok = [](const xinfer_view4 &t) {
    if (t.data == nullptr || (reinterpret_cast<uintptr_t>(t.data) & 15u) != 0 || t.stride[3] != 1) return false;
    for (int i = 0; i < 3; ++i)
      if (t.size[i] > 1 && t.stride[i] % 8 != 0) return false;
    return true;
  };
  for (const xinfer_view4 *t : {q, key, value, cos, sin})
    if (!rows_ok(*t)) return XINFER_ERR_LAYOUT;
  for (const void *p : {q_weight, k_weight, static_cast<const void *>(q_out)})
    if ((reinterpret_cast<uintptr_t>(p) & 15u) != 0) return XINFER_ERR_LAYOUT;
  for (const xinfer_view4 *c : {cache_key, cache_value}) {
    if (!c->data || (reinterpret_cast<uintptr_t>(c->data) & 15u) != 0 || c->size[0] < B || c->size[1] != Hkv ||
        c->size[3] != D || c->size[2] <= 0)
      return XINFER_ERR_CACHE;
    if (c->stride[3] != 1 || c->stride[2] != D || c->stride[1] != c->size[2] * D ||
        c->stride[0] != Hkv * c->size[2] * D)
      return XINFER_ERR_CACHE;
    for (int i = 0; i < 4; ++i)
      if (c->size[i] != cache_key->size[i]) return XINFER_ERR_CACHE;
  }
  NormRopeArgs a{};
  a.q = view_of(*q);
  a.k = view_of(*key);
  a.v = view_of(*value);
  a.q_weight = static_cast<const uint16_t *>(q_weight);
  a.k_weight = static_cast<const uint16_t *>(k_weight);
  a.cos = view_of(*cos);
  a.sin = view_of(*sin);
  a.positions = positions;
  a.pos_sb = pos_stride_b;
  a.pos_st = pos_stride_t;
  a.cu_query = cu_query;
  a.q_out = static_cast<uint16_t *>(q_out);
  a.cache_key = static_cast<uint16_t *>(const_cast<void *>(cache_key->data));
  a.cache_value = static_cast<uint16_t *>(const_cast<void *>(cache_value->data));
  a.eps = (float)eps;
  a.B = (int32_t)B;
  a.T = (int32_t)T;
  a.Hq = (int32_t)Hq;
  a.Hkv = (int32_t)Hkv;
  a.D = (int32_t)D;
  a.C = (int32_t)cache_key->size[2];
  return launch_norm_rope(a, static_cast<hipStream_t>(stream)) == hipSuccess ? XINFER_OK : XINFER_ERR_LAUNCH;
}

int xinfer_projection_gemv(const void *x, const void *weight, void *out, int64_t n, int64_t k, int dtype,
                           void *stream) {
  if (!x || !weight || !out || n <= 0 || k <= 0 || k >= (int64_t(1) << 31) || n >= (int64_t(1) << 31) ||
      (dtype != XINFER_BF16 && dtype != XINFER_FP32))
    return XINFER_ERR_ARGUMENT;
  const int64_t size = dtype == XINFER_FP32 ? 4 : 2;
  const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && (reinterpret_cast<uintptr_t>(weight) & 15u) == 0 &&
                   (k * size) % 16 == 0;
  GemvArgs a{x, weight, out, n, k};
  return launch_gemv(a, dtype == XINFER_FP32, vec, static_cast<hipStream_t>(stream)) == hipSuccess
             ? XINFER_OK
             : XINFER_ERR_LAUNCH;
}

}  // extern "C"
