"""In-place KV-cache append: each row's real new tokens go to their cache positions.

Python entry of the native ``xinfer::append_kv_batched`` operator, with the
reference's name and argument order (compiler/common/kernels/kv_cache.py:45-72).
The operator is registered by libxinfer_attention_ops.so (a HIP kernel, not a
Triton op); calling this function loads the library on first use.
"""

from xinfer_amd.attention import load_attention_ops


def append_kv_batched(key, value, positions, cu_query, cache_key, cache_value):
    """cache_key[r,h,positions[r,t],:] = key[r,h,t,:] (same for value), t < count_r.

    ``key``/``value``: bf16 [B,Hkv,T,D] (any strides); ``positions``: int64
    [B,T]; ``cu_query``: int32 [B+1] cumulative real-token counts on the device
    (``cuda_offsets[0]``); caches: contiguous bf16 [B,Hkv,C,D], mutated in place.
    Positions of padded tokens are not used.  Returns None.
    """
    import torch

    if not hasattr(torch.ops.xinfer, "append_kv_batched"):
        load_attention_ops(model="qwen3")
    torch.ops.xinfer.append_kv_batched(key, value, positions, cu_query, cache_key, cache_value)
