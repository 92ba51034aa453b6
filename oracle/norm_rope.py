"""Numpy restatement of the step before the attention operator -- TEST INFRASTRUCTURE ONLY.

Only tests/ and bench.py use this module, and only as the checker; the
product path (xinfer_amd) never imports it.

What it restates: the eager sequence of compiler/qwen3/adapters/attention.py:44-51
in the reference, i.e.

* ``rms_norm``: transformers' Qwen3RMSNorm.forward (the q_norm / k_norm
  modules of Qwen3Attention, applied per head over the head dimension):
  y = bf16(x * rsqrt(mean(x^2) + eps)) in fp32, then bf16(weight * y);
* ``rope``: transformers' apply_rotary_pos_emb with rotate_half,
  x' = x * cos + rotate_half(x) * sin on bf16 tensors, every product and the
  sum rounded to bf16 as eager PyTorch rounds them;
* ``norm_rope_append``: both, the query returned as [B, Hq, T, D] (the
  adapter's ``transpose(1, 2)``), and the key and value appended as
  compiler/common/kernels/kv_cache.py:8-42 (via KVCache.update,
  compiler/qwen3/model.py:49-52) appends them: only tokens t < count_r, at
  positions[r, t].

bf16 values are handled as uint16 bit patterns; rounding is
round-to-nearest-even.  mean(x^2) is a float32 sum in numpy's order, and the
reciprocal square root is 1 / sqrt in float32: either may differ in its last
bit from another implementation, so results agree with the eager modules to
one bf16 unit in the last place (tests/test_norm_rope.py measures how often).

Pinning (tests/test_norm_rope.py): the rope stage bit for bit against
transformers' apply_rotary_pos_emb on CPU tensors; the norm stage against
Qwen3RMSNorm on CPU tensors within one unit in the last place; closed forms
(a constant row normalises to the weight; cos = 1, sin = 0 is the identity;
cos = 0, sin = 1 is rotate_half); planted mistakes (rotation sign, missing
weight, missing epsilon, wrong half pairing) that must fail; a brute-force
loop for the append.
"""

from __future__ import annotations

import numpy as np


def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """Round-to-nearest-even float32 -> bf16 bits (finite inputs)."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def round_bf16(x):
    return bf16_to_f32(f32_to_bf16(x))


def rms_norm(x_bits, w_bits, eps):
    """Qwen3RMSNorm over the last axis; bf16 bits in, bf16 bits out."""
    x = bf16_to_f32(x_bits)
    var = np.mean(x * x, axis=-1, keepdims=True, dtype=np.float32)
    inv = np.float32(1.0) / np.sqrt(var + np.float32(eps), dtype=np.float32)
    y = round_bf16(x * inv)
    return f32_to_bf16(bf16_to_f32(w_bits) * y)


def rope(x_bits, cos_bits, sin_bits):
    """apply_rotary_pos_emb for one tensor; cos/sin broadcast against x."""
    x = bf16_to_f32(x_bits)
    half = x.shape[-1] // 2
    rot = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    a = round_bf16(x * bf16_to_f32(cos_bits))
    b = round_bf16(rot * bf16_to_f32(sin_bits))
    return f32_to_bf16(a + b)


def norm_rope_append(q, key, value, q_weight, k_weight, eps, cos, sin, positions, cu_query, cache_key,
                     cache_value):
    """The fused step on bf16 bit arrays.

    q [B, T, Hq, D], key/value [B, T, Hkv, D], weights [D], cos/sin [B, T, D],
    positions [B, T], cu_query [B + 1]; caches [B, Hkv, C, D] are updated in
    place.  Returns the rotated query [B, Hq, T, D].
    """
    cs, sn = cos[:, :, None, :], sin[:, :, None, :]
    q_out = rope(rms_norm(q, q_weight, eps), cs, sn)
    k_out = rope(rms_norm(key, k_weight, eps), cs, sn)
    batch, tokens = q.shape[:2]
    capacity = cache_key.shape[2]
    for r in range(batch):
        count = min(max(int(cu_query[r + 1]) - int(cu_query[r]), 0), tokens)
        for t in range(count):
            position = int(positions[r, t])
            if 0 <= position < capacity:
                cache_key[r, :, position, :] = k_out[r, t]
                cache_value[r, :, position, :] = value[r, t]
    return np.ascontiguousarray(q_out.transpose(0, 2, 1, 3))
