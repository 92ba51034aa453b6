"""Numpy restatement of the xinfer attention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py (its cpu_baseline leg) use
this module, and only as the checker; the product path (xinfer_amd) never
imports it.

What it restates (reference files under /root/reference):

* ``attention``: compiler/common/kernels/attention.cpp:14-79
  (xinfer::batched_flash_attention) -- row r attends with its first count_r
  queries over K/V[r, :, :L_r] with lower-right causality (query i sees keys
  j <= L_r - count_r + i, docs/flash-attention.md:15 and the mask of
  compiler/common/tests/test_attention.py:95-98), grouped-query heads
  (query head hq uses KV head hq // (Hq/Hkv), ATen's enable_gqa mapping used
  by the reference tests), softmax(scale * q.k) v, and zeros for the padded
  queries t >= count_r (attention.cpp:54,73-77).
* ``flash_attention``: attention.cpp:82-124 -- the same math with count = T
  and one valid length L for every row (kv_extent carries only L + 1 as its
  length, compiler/common/attention.py:20-24).
* ``append_kv``: compiler/common/kernels/kv_cache.py:8-42 --
  cache[r, h, positions[r, t], :] = new[r, h, t, :] for t < count_r, with
  count_r = cu_query[r+1] - cu_query[r]; padded positions never read.
* ``batched_metadata``: compiler/common/attention.py:27-40 -- cumulative sums.

Floating point: the oracle computes in float64 by default (the reference tests'
bound is an fp32 SDPA MATH reference, compiler/common/tests/test_attention.py:99-107);
``dtype=np.float32`` is the faster variant timed as the CPU baseline.

Pinning (tests/test_oracle.py): the reference's known-answer test
(test_attention.py:293-306, outputs [1.5, 2.0]), torch's SDPA MATH backend
with an explicit lower-right mask and enable_gqa (the reference tests' own
oracle), an explicit triple-loop softmax on tiny inputs, closed forms
(one visible key -> its value; equal scores -> running mean), a GQA head
mapping check, and brute-force loops for the append and the metadata.
"""

from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------------------- bf16 bits


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bit patterns (uint16) to float32."""
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 bits, nearest-even (NaN kept quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), rounded)
    return rounded


# ----------------------------------------------------------------------------- attention


def attention(q, k, v, counts, lengths, scale, dtype=np.float64):
    """Batched valid-prefix attention (attention.cpp:14-79).

    q: [B, Hq, T, D]; k, v: [B, Hkv, C, D] (float arrays: bf16 values widened
    exactly); counts, lengths: per-row real queries and populated KV lengths.
    Returns [B, Hq, T, D] in ``dtype``; rows t >= counts[r] are zero.
    """
    q = np.asarray(q)
    k = np.asarray(k)
    v = np.asarray(v)
    batch, heads, tokens, dim = q.shape
    kv_heads = k.shape[1]
    if heads % kv_heads:
        raise ValueError("Query heads must be a positive multiple of KV heads")
    group = heads // kv_heads
    out = np.zeros((batch, heads, tokens, dim), dtype=dtype)
    for r in range(batch):
        count, length = int(counts[r]), int(lengths[r])
        if not 0 <= count <= tokens or not count <= length <= k.shape[2] or length < 1:
            raise ValueError("Invalid query/KV lengths")
        if count == 0:
            continue
        # Query i (0-based) sees keys j <= length - count + i.
        visible = np.arange(length)[None, :] <= (length - count + np.arange(count))[:, None]
        for hq in range(heads):
            h = hq // group
            qr = q[r, hq, :count].astype(dtype)
            kr = k[r, h, :length].astype(dtype)
            vr = v[r, h, :length].astype(dtype)
            scores = (qr @ kr.T) * dtype(scale)
            scores = np.where(visible, scores, -np.inf)
            scores -= scores.max(axis=1, keepdims=True)
            weights = np.exp(scores)
            weights /= weights.sum(axis=1, keepdims=True)
            out[r, hq, :count] = weights @ vr
    return out


def flash_attention(q, k, v, valid_length, scale, dtype=np.float64):
    """Uniform-length prefix attention (attention.cpp:82-124): count = T for every row."""
    batch, tokens = q.shape[0], q.shape[2]
    if not tokens <= valid_length <= k.shape[2]:
        raise ValueError("Invalid valid-prefix length")
    return attention(q, k, v, [tokens] * batch, [valid_length] * batch, scale, dtype=dtype)


# ----------------------------------------------------------------------------- append


def append_kv(cache_key, cache_value, key, value, positions, cu_query):
    """In-place KV append (kv_cache.py:8-42) on uint16 bf16 bit arrays.

    cache_*: [B, H, C, D]; key/value: [B, H, T, D]; positions: int [B, T];
    cu_query: int [B+1].  Positions of padded tokens (t >= count_r) are not read.
    """
    batch, heads, tokens, _ = key.shape
    for r in range(batch):
        count = int(cu_query[r + 1]) - int(cu_query[r])
        for t in range(min(max(count, 0), tokens)):
            position = int(positions[r, t])
            cache_key[r, :, position, :] = key[r, :, t, :]
            cache_value[r, :, position, :] = value[r, :, t, :]


# ----------------------------------------------------------------------------- metadata


def batched_metadata(kv_lengths, query_lengths):
    """CPU offsets [2, B+1] of batched_attention_metadata (attention.py:27-40)."""
    lengths = np.stack([np.asarray(query_lengths), np.asarray(kv_lengths)]).astype(np.int64)
    offsets = np.zeros((2, lengths.shape[1] + 1), dtype=np.int32)
    offsets[:, 1:] = np.cumsum(lengths, axis=1)
    return offsets
