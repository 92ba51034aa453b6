/*
 * C ABI of libxinfer_attention_ops.so: attention over each request's populated
 * KV prefix and the in-place KV-cache append, for AMD MI355X (gfx950).
 *
 * Every entry point takes plain device pointers, element strides and host-side
 * lengths; none allocates device memory and none synchronises the host with the
 * device.  Work is enqueued on `stream` (a hipStream_t; NULL is the null stream).
 * Tensors are bf16 (stored as raw uint16 bits).  Return value: 0 on success, or
 * a status code whose message `xinfer_status_string` returns.  The messages
 * reproduce the reference operator's TORCH_CHECK texts where one exists.
 *
 * The torch.library operators and the AOTInductor C shims that the reference
 * exports are defined in the same library; they validate torch-specific
 * properties and call the entry points below.
 */
#ifndef XINFER_ATTENTION_H
#define XINFER_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes.  Messages (xinfer_status_string) follow the reference:
 * compiler/common/kernels/attention.cpp:17-35 and :84-104. */
enum {
  XINFER_OK = 0,
  XINFER_ERR_QKV_SHAPES = 1,      /* "Invalid Q/K/V shapes"                        attention.cpp:17-19 */
  XINFER_ERR_Q_SHAPE = 2,         /* "Unsupported Q shape"                         attention.cpp:90-91 */
  XINFER_ERR_KV_SHAPE = 3,        /* "Expected matching full-capacity K/V ..."     attention.cpp:92-94 */
  XINFER_ERR_HEADS = 4,           /* "Query heads must be a positive multiple ..." attention.cpp:95-96 */
  XINFER_ERR_HEAD_DIM = 5,        /* "Flash head dimension must be ..."            attention.cpp:97-98 */
  XINFER_ERR_PREFIX = 6,          /* "Invalid valid-prefix length"                 attention.cpp:102 */
  XINFER_ERR_SCALE = 7,           /* "Attention scale must be finite and positive" attention.cpp:103 */
  XINFER_ERR_OFFSETS_START = 8,   /* "Cumulative lengths must start at zero"       attention.cpp:35 */
  XINFER_ERR_LENGTHS = 9,         /* "Invalid query/KV lengths"                    attention.cpp:43-45 */
  XINFER_ERR_WORKSPACE = 10,      /* workspace smaller than its *_workspace_size, or not 16-byte aligned */
  XINFER_ERR_LAYOUT = 11,         /* feature stride != 1 or rows not 16-byte aligned */
  XINFER_ERR_CACHE = 12,          /* cache tensors not contiguous [B,H,C,D] / shape mismatch */
  XINFER_ERR_LAUNCH = 13,         /* a HIP kernel launch failed */
  XINFER_ERR_ARGUMENT = 14,       /* null pointer, negative size or stride, misaligned page table */
  XINFER_ERR_ROPE_SHAPE = 15,     /* xinfer_qk_norm_rope_append shapes (no reference message) */
  XINFER_ERR_EPS = 16,            /* RMSNorm epsilon not finite and >= 0 (no reference message) */
  XINFER_ERR_SCRATCH = 17,        /* the call needs more than XINFER_NOALLOC_SCRATCH_BYTES of scratch */
  XINFER_ERR_CAPTURE_ROWS = 18    /* graph-capture mode: more than 64 rows */
};

/* A strided rank-4 view of bf16 device memory, [batch, heads, sequence, dim].
 * Strides are in elements.  The attention kernels need stride[3] == 1, the
 * other strides multiples of 8 and `data` 16-byte aligned (XINFER_ERR_LAYOUT
 * otherwise); the append kernel accepts any strides for key/value. */
typedef struct xinfer_view4 {
  const void *data;
  int64_t size[4];
  int64_t stride[4];
} xinfer_view4;

/* Message for a status code (static storage, never NULL). */
const char *xinfer_status_string(int status);

/* ---------------------------------------------------------------------------
 * xinfer::flash_attention -- replaces compiler/common/kernels/attention.cpp:82-124
 * (schema :133-134, fake compiler/common/attention.py:63-83).
 *
 * q [B,Hq,T,D], k/v [B,Hkv,C,D]; every row attends with all T queries over the
 * first `valid_length` cache positions, lower-right causal: query i sees keys
 * j <= valid_length - T + i.  out: contiguous [B,Hq,T,D] bf16, written fully.
 * ------------------------------------------------------------------------- */
size_t xinfer_flash_attention_workspace_size(const xinfer_view4 *q, const xinfer_view4 *k,
                                             int64_t valid_length);
int xinfer_flash_attention(const xinfer_view4 *q, const xinfer_view4 *k, const xinfer_view4 *v,
                           int64_t valid_length, double scale, void *out, void *workspace,
                           size_t workspace_bytes, void *stream);

/* ---------------------------------------------------------------------------
 * xinfer::batched_flash_attention -- replaces attention.cpp:14-79
 * (schema :129-131, fake compiler/common/attention.py:86-94).
 *
 * host_offsets: host int32 [2][B+1]; row 0 = cumulative real-query counts,
 * row 1 = cumulative populated KV lengths (both start at 0), exactly the CPU
 * `offsets` tensor of batched_attention_metadata (attention.py:27-40).  Row r
 * attends with its first count_r queries over k/v[r, :, :L_r], lower-right
 * causal; out[r, :, count_r:] is written as zeros.
 *
 * blocks: NULL, or the DEVICE int32 page table of attention.cpp:39-40, 56-58,
 * 68-70, one entry per row at blocks[r * blocks_stride] (blocks_stride >= 0,
 * the table's row stride; 4-byte aligned): row r then reads its keys and
 * values from k/v[blocks[r]] instead of k/v[r], each entry clamped into
 * [0, B).  The reference applies its table only when the cache capacity C is
 * a multiple of 256; xinfer::batched_flash_attention passes it under that
 * condition and NULL otherwise.  The kernels read it on the device: the
 * identity table costs one scalar read per work item.
 * ------------------------------------------------------------------------- */
size_t xinfer_batched_flash_attention_workspace_size(const xinfer_view4 *q, const xinfer_view4 *k,
                                                     const int32_t *host_offsets);
int xinfer_batched_flash_attention(const xinfer_view4 *q, const xinfer_view4 *k,
                                   const xinfer_view4 *v, const int32_t *host_offsets,
                                   const int32_t *blocks, int64_t blocks_stride, double scale,
                                   void *out, void *workspace, size_t workspace_bytes, void *stream);

/* Same operation with the output written through a caller-supplied view of
 * q's sizes [B,Hq,T,D] (unit feature stride, other strides multiples of 8,
 * 16-byte aligned data), e.g. [B,T,Hq,D] storage viewed as [B,Hq,T,D].  The
 * view's elements must be distinct and must not overlap q, k, v or the
 * workspace.  The workspace is the one *_workspace_size reports.  No reference counterpart:
 * it serves xinfer::batched_flash_attention_bthd, the optional variant that
 * spares compiler/qwen3/adapters/attention.py:61 its transpose copy. */
int xinfer_batched_flash_attention_out(const xinfer_view4 *q, const xinfer_view4 *k,
                                       const xinfer_view4 *v, const int32_t *host_offsets,
                                       const int32_t *blocks, int64_t blocks_stride,
                                       double scale, const xinfer_view4 *out, void *workspace,
                                       size_t workspace_bytes, void *stream);

/* Graph-capture ("capture once, replay every step") variant of
 * xinfer_batched_flash_attention.  No counterpart in the reference, which
 * leaves graph capture to future runtime work (PLAN.md:35-37): it is for
 * serving loops that capture one step in a HIP graph and replay it while the
 * lengths change.  device_offsets is the DEVICE copy of
 * the cumulative offsets (int32 [2][B+1], batched_attention_metadata's
 * cuda_offsets); the kernels read every row's count and length from it when
 * they run, so nothing about the launch depends on host lengths and a
 * captured call stays valid after the caller rewrites device_offsets in place
 * (and the page table, read the same way).
 * The workspace size depends on the shapes only (all rows at capacity C).
 * Shapes with T * (Hq/Hkv) <= 8 take the decode kernels; larger ones take the
 * prefill kernels, whose key split size, work list and XCD runs a plan kernel
 * chooses from device_offsets at run time and writes into the workspace (at
 * most 8 splits a row; the workspace holds records for the most items such a
 * plan can make).  B <= 64 (XINFER_ERR_CAPTURE_ROWS otherwise).  Device lengths are not validated on
 * the host: counts are clamped to [0, min(T, C)] and lengths to [max(count, 1), C], so
 * bad values give wrong rows but never an access outside the tensors.
 * Results agree with xinfer_batched_flash_attention within rounding; the
 * kernels are the same, but every launch covers the capacity. */
size_t xinfer_batched_flash_attention_graph_workspace_size(const xinfer_view4 *q, const xinfer_view4 *k);
int xinfer_batched_flash_attention_graph(const xinfer_view4 *q, const xinfer_view4 *k, const xinfer_view4 *v,
                                         const int32_t *device_offsets, const int32_t *blocks,
                                         int64_t blocks_stride, double scale, void *out, void *workspace,
                                         size_t workspace_bytes, void *stream);

/* Allocation-free variant of xinfer_batched_flash_attention.  No counterpart in
 * the reference: it is for callers that cannot allocate device memory or pass
 * a workspace -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  Same arguments, checks, kernels and results as
 * xinfer_batched_flash_attention, bit for bit; the split records go to a
 * static device array of the library (one per GPU, held until the process
 * ends) instead of a caller's workspace, and the call allocates nothing.
 * A call whose records exceed XINFER_NOALLOC_SCRATCH_BYTES (the size
 * xinfer_batched_flash_attention_workspace_size reports) returns
 * XINFER_ERR_SCRATCH and launches nothing.  The current device must be the
 * stream's.  Calls that overlap in time on one GPU share its array and race:
 * order them on one stream. */
#define XINFER_NOALLOC_SCRATCH_BYTES (32u << 20)
int xinfer_batched_flash_attention_noalloc(const xinfer_view4 *q, const xinfer_view4 *k,
                                           const xinfer_view4 *v, const int32_t *host_offsets,
                                           const int32_t *blocks, int64_t blocks_stride,
                                           double scale, void *out, void *stream);

/* ---------------------------------------------------------------------------
 * xinfer::append_kv_batched -- replaces the Triton op
 * compiler/common/kernels/kv_cache.py:8-72.
 *
 * cache_key[r,h,positions[r,t],:] = key[r,h,t,:] (same for value) for
 * t < count_r = cu_query[r+1] - cu_query[r]; positions of padded tokens are
 * not used (they are loaded with the rest, so every one of the B*T entries
 * must be readable).  positions: device int64 [B,T] with strides
 * (pos_stride_b, pos_stride_t); cu_query: device int32 [B+1].  Caches are contiguous
 * [B,Hkv,C,D] bf16 and are the only memory written.  A position outside
 * [0, C) is skipped instead of being written out of bounds.
 * ------------------------------------------------------------------------- */
int xinfer_append_kv_batched(const xinfer_view4 *key, const xinfer_view4 *value,
                             const int64_t *positions, int64_t pos_stride_b, int64_t pos_stride_t,
                             const int32_t *cu_query, const xinfer_view4 *cache_key,
                             const xinfer_view4 *cache_value, void *stream);

/* ---------------------------------------------------------------------------
 * xinfer::qk_norm_rope_append -- replaces the eager step before the attention
 * operator, compiler/qwen3/adapters/attention.py:44-51 (q_norm/k_norm, i.e.
 * transformers Qwen3RMSNorm, then apply_rotary_pos_emb, then
 * KVCache.update = append_kv_batched, compiler/qwen3/model.py:49-52).
 *
 * q [B,Hq,T,D], key/value [B,Hkv,T,D]: projections viewed per head (any
 * strides with unit feature stride, others divisible by 8, 16-byte aligned);
 * q_weight/k_weight: the [D] RMSNorm weights; cos/sin [B,1,T,D] (stride[1]
 * unused): the rotary tables of the tokens; D in {64, 128, 256}.
 *   xn = bf16(w * bf16(x * rsqrt(mean(x^2) + eps)))   per (token, head) row
 *   x' = bf16(bf16(xn * cos) + bf16(rotate_half(xn) * sin))
 * q_out: contiguous [B,Hq,T,D] receives q' for every token.  cache_key
 * receives k' and cache_value v at [r, h, positions[r,t]] for t < count_r
 * (count_r, positions and the skipping of positions outside [0, C) as in
 * xinfer_append_kv_batched).  No reference counterpart in the C ABI: the
 * reference runs this step as separate eager or compiled PyTorch ops.
 * ------------------------------------------------------------------------- */
int xinfer_qk_norm_rope_append(const xinfer_view4 *q, const xinfer_view4 *key, const xinfer_view4 *value,
                               const void *q_weight, const void *k_weight, double eps,
                               const xinfer_view4 *cos, const xinfer_view4 *sin, const int64_t *positions,
                               int64_t pos_stride_b, int64_t pos_stride_t, const int32_t *cu_query,
                               void *q_out, const xinfer_view4 *cache_key, const xinfer_view4 *cache_value,
                               void *stream);

/* ---------------------------------------------------------------------------
 * xinfer::projection_gemv -- replaces the Triton op
 * compiler/common/kernels/projection_gemv.py:10-62 (the decoder's singleton
 * projections, selected by compiler/common/passes/projection_gemv.py).
 *
 * out[i] = sum_j weight[i, j] * x[j] for i < n, j < k: x [k] contiguous,
 * weight [n, k] contiguous row-major, out [n]; all XINFER_BF16 or all
 * XINFER_FP32 (dtype), accumulated in fp32.  out must not overlap x or weight.
 * ------------------------------------------------------------------------- */
enum { XINFER_BF16 = 0, XINFER_FP32 = 1 };
int xinfer_projection_gemv(const void *x, const void *weight, void *out, int64_t n, int64_t k, int dtype,
                           void *stream);

/* The AOTInductor C shims of the same library are declared in
 * xinfer_attention_aoti.h. */

#ifdef __cplusplus
}
#endif

#endif /* XINFER_ATTENTION_H */
