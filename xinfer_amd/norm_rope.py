"""The step before the attention operator as one native launch.

Python entry of ``xinfer::qk_norm_rope_append`` (libxinfer_attention_ops.so,
HIP kernel xinfer_amd/csrc/norm_rope.hip).  It replaces this eager sequence of
the reference's Qwen3 adapter (compiler/qwen3/adapters/attention.py:44-51):

    q = q_norm(q_proj(x).view(B, T, Hq, D)).transpose(1, 2)
    k = k_norm(k_proj(x).view(B, T, Hkv, D)).transpose(1, 2)
    v = v_proj(x).view(B, T, Hkv, D).transpose(1, 2)
    q, k = apply_rotary_pos_emb(q, k, cos, sin)
    k, v = past_key_value.update(k, v, ...)      # append_kv_batched

with the same arithmetic and bf16 rounding points (transformers Qwen3RMSNorm,
apply_rotary_pos_emb), so that the attention operator sees the same query and
cache contents.  The attention call itself is unchanged.
"""

from xinfer_amd.attention import load_attention_ops


def qk_norm_rope_append(q, key, value, q_weight, k_weight, eps, cos, sin, positions, cu_query, cache_key,
                        cache_value):
    """Normalise, rotate and append; returns the rotated query [B,Hq,T,D].

    ``q`` bf16 [B,T,Hq,D] and ``key``/``value`` bf16 [B,T,Hkv,D]: the
    projections viewed per head; ``q_weight``/``k_weight``: the [D] RMSNorm
    weights and ``eps`` their epsilon; ``cos``/``sin`` bf16 [B,T,D]: the
    rotary tables of the tokens (``position_embeddings``); ``positions`` int64
    [B,T] and ``cu_query`` int32 [B+1] as for ``append_kv_batched``; caches
    contiguous bf16 [B,Hkv,C,D], mutated in place for the real tokens
    (t < count_r) only.  The returned query is contiguous.
    """
    import torch

    if not hasattr(torch.ops.xinfer, "qk_norm_rope_append"):
        load_attention_ops(model="qwen3")
    return torch.ops.xinfer.qk_norm_rope_append(q, key, value, q_weight, k_weight, float(eps), cos, sin, positions,
                                                cu_query, cache_key, cache_value)
