// Host-side launchers of the HIP kernels (defined in the .hip files).
#pragma once

#include <hip/hip_runtime_api.h>

#include "kernel_args.h"

namespace xattn {

hipError_t launch_append(const AppendArgs &a, bool vector, hipStream_t stream);
hipError_t launch_norm_rope(const NormRopeArgs &a, hipStream_t stream);
// fp32: float inputs and output, else bf16; vec: 16-byte aligned rows and input.
hipError_t launch_gemv(const GemvArgs &a, bool fp32, bool vec, hipStream_t stream);

// Keys of one decode round for padded head dim `dp` and `qr` query vectors per
// KV head (a power of two <= 8); an item of `rounds` rounds (1 or
// kDecodeItemRounds) takes rounds times as many.
constexpr int kDecodeItemRounds = 4;
int decode_tokens_per_item(int dp, int qr);
hipError_t launch_decode(const AttnArgs &a, int dp, int qr, int rounds, int items, hipStream_t stream);

hipError_t launch_prefill(const AttnArgs &a, int dp, hipStream_t stream);
// The head-dim-256 prefill kernel over `blocks` blocks (prefill_d256.hip).
hipError_t launch_prefill_d256(const AttnArgs &a, unsigned blocks, hipStream_t stream);
// Graph-capture prefill: the plan kernel writes *p.attn and *p.merge from the
// device offsets, then the prefill kernel runs over `blocks` blocks with its
// arguments read from *p.attn (blocks past their XCD run exit).
hipError_t launch_prefill_capture(const PrefillPlanArgs &p, int dp, unsigned blocks, hipStream_t stream);
hipError_t launch_prefill_d256_dev(const AttnArgs *a, unsigned blocks, hipStream_t stream);
// The merge with its arguments in device memory (written by the plan
// kernel): grid for up to max_vectors query vectors; max_splits picks the
// thread layout.
hipError_t launch_merge_dev(const MergeArgs *a, int dp, int max_splits, int64_t max_vectors, hipStream_t stream);

// Merges a.total_items query vectors; max_splits picks the thread layout.
hipError_t launch_merge(const MergeArgs &a, int dp, int max_splits, hipStream_t stream);
// Splits per query vector up to which the merge gives each (vector, 4
// features) one thread that folds the splits in increasing order.  The decode
// kernel's in-launch merge serves only such launches and folds the same way.
constexpr int kMergeSerialSplits = 8;

// Whether the device gives consecutive blocks of a launch to its 8 XCDs in
// turn (block b on the XCD of block b % 8), which the decode kernel's
// in-launch merge relies on: a small probe launch, synchronised on `stream`.
hipError_t probe_xcd_dispatch(bool *round_robin, hipStream_t stream);

// Graph-capture decode: the decode kernel over `blocks` blocks, then the merge
// of every query vector of the capacity layout; max_splits = splits of a
// row at capacity picks the merge's thread layout.
hipError_t launch_decode_capture(const CaptureArgs &c, int dp, int qr, int rounds, int blocks, hipStream_t stream);
hipError_t launch_merge_capture(const CaptureArgs &c, int dp, int max_splits, hipStream_t stream);

// Bytes of the static device scratch behind the allocation-free entry point
// (XINFER_NOALLOC_SCRATCH_BYTES of the C header).
constexpr size_t kScratchBytes = size_t(32) << 20;
// The current device's address of that scratch (scratch.hip), looked up once
// per device.
hipError_t scratch_pointer(void **pointer);

}  // namespace xattn
