/*
 * AOTInductor C shims exported by libxinfer_attention_ops.so.
 *
 * These are the symbols a generated AOTI wrapper.cpp calls directly when
 * torch._inductor.config.aot_inductor.custom_ops_to_c_shims maps the xinfer
 * operators to them (compiler/common/package.py:55-78).  Input handles are
 * borrowed; the output handle is a new tensor whose ownership passes to the
 * caller.  Errors (the operators' TORCH_CHECK messages) are reported as
 * AOTI_TORCH_FAILURE with the message stored by torch's error bridge.
 *
 * The handle types are the opaque ones of torch/csrc/inductor/aoti_torch/c/shim.h.
 */
#ifndef XINFER_ATTENTION_AOTI_H
#define XINFER_ATTENTION_AOTI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
struct AtenTensorOpaque;
typedef AtenTensorOpaque *AtenTensorHandle;
#else
typedef struct AtenTensorOpaque *AtenTensorHandle;
#endif
typedef int32_t AOTITorchError;

/* Replaces compiler/common/kernels/attention_shim.cpp:21-32 (declared as a
 * string at compiler/common/attention.py:10-12). */
AOTITorchError aoti_torch_cuda_flash_attention(AtenTensorHandle q, AtenTensorHandle k,
                                               AtenTensorHandle v, AtenTensorHandle extent,
                                               double scale, AtenTensorHandle *output);

/* Replaces compiler/common/kernels/attention_shim.cpp:5-19 (declared as a
 * string at compiler/common/attention.py:13-16). */
AOTITorchError aoti_torch_cuda_batched_flash_attention(AtenTensorHandle q, AtenTensorHandle k,
                                                       AtenTensorHandle v, AtenTensorHandle offsets,
                                                       AtenTensorHandle cuda_offsets,
                                                       AtenTensorHandle blocks, double scale,
                                                       AtenTensorHandle *output);

/* New, optional: xinfer::batched_flash_attention_bthd, the same operation
 * with a contiguous [B,T,Hq,D] output (xinfer_batched_flash_attention_out). */
AOTITorchError aoti_torch_cuda_batched_flash_attention_bthd(AtenTensorHandle q, AtenTensorHandle k,
                                                            AtenTensorHandle v, AtenTensorHandle offsets,
                                                            AtenTensorHandle cuda_offsets,
                                                            AtenTensorHandle blocks, double scale,
                                                            AtenTensorHandle *output);

/* New: the reference's append is a Triton op (compiler/common/kernels/kv_cache.py:45-72)
 * that AOTI compiles into the wrapper; the native op needs its own shim.  It
 * mutates cache_key/cache_value in place and returns nothing.  AOTInductor's
 * wrapper passes one output slot for the operator's empty result, always
 * null; it is never written. */
AOTITorchError aoti_torch_cuda_append_kv_batched(AtenTensorHandle key, AtenTensorHandle value,
                                                 AtenTensorHandle positions,
                                                 AtenTensorHandle cu_query,
                                                 AtenTensorHandle cache_key,
                                                 AtenTensorHandle cache_value,
                                                 AtenTensorHandle *unused_output);

/* New: the fused step before the attention operator (xinfer_qk_norm_rope_append
 * in xinfer_attention.h), which replaces eager ops of
 * compiler/qwen3/adapters/attention.py:44-51 that AOTI would otherwise compile
 * into the wrapper.  Returns the rotated query [B,Hq,T,D] as a new tensor and
 * mutates cache_key/cache_value in place. */
AOTITorchError aoti_torch_cuda_qk_norm_rope_append(
    AtenTensorHandle q, AtenTensorHandle key, AtenTensorHandle value, AtenTensorHandle q_weight,
    AtenTensorHandle k_weight, double eps, AtenTensorHandle cos, AtenTensorHandle sin,
    AtenTensorHandle positions, AtenTensorHandle cu_query, AtenTensorHandle cache_key,
    AtenTensorHandle cache_value, AtenTensorHandle *output);

/* New: the native xinfer::projection_gemv (replaces the Triton op
 * compiler/common/kernels/projection_gemv.py:35-62, which AOTI compiled into
 * the wrapper).  Returns the new [*x.shape[:-1], n] output. */
AOTITorchError aoti_torch_cuda_projection_gemv(AtenTensorHandle x, AtenTensorHandle weight,
                                               AtenTensorHandle *output);

#ifdef __cplusplus
}
#endif

#endif /* XINFER_ATTENTION_AOTI_H */
