"""Pin the CPU oracle (oracle/attention.py) before anything is checked against it.

Each check is chosen so a plausible mistake fails it: the reference's
known-answer test fixes the causal direction, torch's SDPA MATH backend (the
reference tests' own oracle, compiler/common/tests/test_attention.py:99-107)
fixes the whole formula, the triple loop restates softmax independently, and
the closed forms fix the head mapping, masking and scaling separately.  The
last test plants those mistakes into copies of the oracle and shows the checks
catch them.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from oracle import attention as oracle

GEOMETRIES = ((16, 8, 128), (8, 2, 256), (16, 4, 256), (6, 2, 64))


def random_case(rng, batch, heads, kv_heads, dim, tokens, capacity):
    q = rng.standard_normal((batch, heads, tokens, dim))
    k = rng.standard_normal((batch, kv_heads, capacity, dim))
    v = rng.standard_normal((batch, kv_heads, capacity, dim))
    return q, k, v


def sdpa_reference(q, k, v, count, length, scale):
    """torch SDPA MATH in float64 with the reference tests' lower-right mask."""
    mask = torch.arange(length)[None, :] <= torch.arange(length - count, length)[:, None]
    with sdpa_kernel(SDPBackend.MATH):
        return F.scaled_dot_product_attention(
            torch.from_numpy(q[:, :, :count]),
            torch.from_numpy(k[:, :, :length]),
            torch.from_numpy(v[:, :, :length]),
            attn_mask=mask,
            enable_gqa=True,
            scale=scale,
        ).numpy()


def kat_inputs(heads, kv_heads, dim):
    """test_attention.py:293-306: q = k = 0, v[j] = j, L = 5, T = 2."""
    q = np.zeros((1, heads, 2, dim))
    k = np.zeros((1, kv_heads, 1024, dim))
    v = np.broadcast_to(np.arange(1024.0)[None, None, :, None], (1, kv_heads, 1024, dim)).copy()
    return q, k, v


def check_kat(function):
    for heads, kv_heads, dim in ((16, 8, 128), (8, 2, 256)):
        out = function(*kat_inputs(heads, kv_heads, dim), 5, dim**-0.5)
        expected = np.array([1.5, 2.0])[None, None, :, None]
        if not np.array_equal(out, np.broadcast_to(expected, out.shape)):
            return False
    return True


def check_sdpa(function, rng):
    for heads, kv_heads, dim in GEOMETRIES:
        for tokens, length in ((1, 1), (1, 37), (3, 3), (5, 29), (16, 40)):
            q, k, v = random_case(rng, 2, heads, kv_heads, dim, tokens, 48)
            out = function(q, k, v, length, dim**-0.5)
            ref = sdpa_reference(q, k, v, tokens, length, dim**-0.5)
            if not np.allclose(out, ref, rtol=0, atol=1e-10):
                return False
    return True


def check_gqa_mapping(function):
    q = np.zeros((1, 4, 1, 8))
    k = np.zeros((1, 2, 4, 8))
    v = np.zeros((1, 2, 4, 8))
    v[0, 0] = 1.0
    v[0, 1] = 2.0
    out = function(q, k, v, 4, 8**-0.5)
    return np.array_equal(out[0, :, 0, 0], [1.0, 1.0, 2.0, 2.0])


def test_known_answer_lower_right_causality():
    assert check_kat(oracle.flash_attention)


def test_matches_torch_sdpa_math_with_lower_right_mask():
    assert check_sdpa(oracle.flash_attention, np.random.default_rng(7))


def test_matches_explicit_triple_loop():
    rng = np.random.default_rng(11)
    heads, kv_heads, dim, tokens, length = 4, 2, 8, 3, 5
    q, k, v = random_case(rng, 1, heads, kv_heads, dim, tokens, 6)
    scale = 0.37
    out = oracle.flash_attention(q, k, v, length, scale)
    for hq in range(heads):
        h = hq // (heads // kv_heads)
        for i in range(tokens):
            last = length - tokens + i
            scores = [scale * sum(q[0, hq, i, d] * k[0, h, j, d] for d in range(dim)) for j in range(last + 1)]
            top = max(scores)
            weights = [math.exp(s - top) for s in scores]
            total = sum(weights)
            for d in range(dim):
                expected = sum(w * v[0, h, j, d] for j, w in enumerate(weights)) / total
                assert abs(out[0, hq, i, d] - expected) < 1e-12


def test_closed_forms():
    rng = np.random.default_rng(3)
    # One visible key: the output is that key's value.
    q, k, v = random_case(rng, 1, 4, 2, 16, 1, 8)
    out = oracle.flash_attention(q, k, v, 1, 0.25)
    assert np.allclose(out[0, :, 0], v[0, [0, 0, 1, 1], 0], atol=1e-15)
    # Identical keys: equal scores, so each query averages its visible values.
    q, k, v = random_case(rng, 1, 4, 2, 16, 3, 8)
    k[:] = k[:, :, :1]
    out = oracle.flash_attention(q, k, v, 6, 0.25)
    for i in range(3):
        visible = 6 - 3 + i + 1
        assert np.allclose(out[0, :, i], v[0, [0, 0, 1, 1], :visible].mean(axis=1), atol=1e-13)
    # GQA: query head hq reads KV head hq // G (not hq % Hkv).
    assert check_gqa_mapping(oracle.flash_attention)
    # Keys past a query's causal limit do not change its output.
    q, k, v = random_case(rng, 1, 4, 2, 16, 4, 12)
    base = oracle.flash_attention(q, k, v, 10, 0.3)
    k2, v2 = k.copy(), v.copy()
    k2[:, :, 7:] = 50.0
    v2[:, :, 7:] = -50.0
    moved = oracle.flash_attention(q, k2, v2, 10, 0.3)
    assert np.array_equal(base[:, :, 0], moved[:, :, 0])  # query 0 sees keys 0..6
    assert not np.allclose(base[:, :, 3], moved[:, :, 3])


def test_batched_rows_padding_and_isolation():
    rng = np.random.default_rng(5)
    q, k, v = random_case(rng, 3, 6, 2, 32, 7, 30)
    counts, lengths = [7, 0, 2], [20, 4, 2]
    out = oracle.attention(q, k, v, counts, lengths, 0.2)
    assert np.count_nonzero(out[0, :, :7]) == out[0, :, :7].size
    assert np.count_nonzero(out[1]) == 0
    assert np.count_nonzero(out[2, :, 2:]) == 0
    # Each row equals the uniform-length operator applied to that row alone.
    for r, (count, length) in enumerate(zip(counts, lengths)):
        if count:
            alone = oracle.flash_attention(q[r:r + 1, :, :count], k[r:r + 1], v[r:r + 1], length, 0.2)
            assert np.array_equal(out[r:r + 1, :, :count], alone)
    with pytest.raises(ValueError, match="Invalid query/KV lengths"):
        oracle.attention(q, k, v, [8, 0, 1], [20, 4, 2], 0.2)


def test_append_matches_loops_and_never_reads_padding():
    rng = np.random.default_rng(9)
    batch, heads, tokens, dim, capacity = 3, 2, 5, 8, 16
    cache_k = rng.integers(0, 2**16, (batch, heads, capacity, dim), dtype=np.uint16)
    cache_v = rng.integers(0, 2**16, (batch, heads, capacity, dim), dtype=np.uint16)
    key = rng.integers(0, 2**16, (batch, heads, tokens, dim), dtype=np.uint16)
    value = rng.integers(0, 2**16, (batch, heads, tokens, dim), dtype=np.uint16)
    counts = [5, 0, 2]
    cu = np.concatenate([[0], np.cumsum(counts)])
    positions = np.full((batch, tokens), capacity + 100)  # out of range unless real
    positions[0] = [3, 4, 5, 6, 7]
    positions[2, :2] = [14, 15]
    expected_k, expected_v = cache_k.copy(), cache_v.copy()
    for r in range(batch):
        for t in range(counts[r]):
            for h in range(heads):
                for d in range(dim):
                    expected_k[r, h, positions[r, t], d] = key[r, h, t, d]
                    expected_v[r, h, positions[r, t], d] = value[r, h, t, d]
    oracle.append_kv(cache_k, cache_v, key, value, positions, cu)
    assert np.array_equal(cache_k, expected_k) and np.array_equal(cache_v, expected_v)
    # torch's index_copy_ agrees on the real rows (the reference packaging test's oracle).
    torch_cache = torch.from_numpy(expected_k[0].astype(np.int32))
    torch_cache.index_copy_(1, torch.tensor(positions[0]), torch.from_numpy(key[0].astype(np.int32)))
    assert np.array_equal(torch_cache.numpy(), cache_k[0].astype(np.int32))


def test_metadata_is_a_cumulative_sum():
    from xinfer_amd.attention import batched_attention_metadata

    kv_lengths, query_lengths = [17, 1, 600, 5], [1, 0, 512, 5]
    offsets = oracle.batched_metadata(kv_lengths, query_lengths)
    for row, lengths in enumerate((query_lengths, kv_lengths)):
        running = 0
        for r, n in enumerate(lengths):
            assert offsets[row, r] == running
            running += n
        assert offsets[row, -1] == running
    host, device, blocks = batched_attention_metadata(
        torch.tensor(kv_lengths, dtype=torch.int32), torch.tensor(query_lengths, dtype=torch.int32), "cpu"
    )
    assert host.dtype == torch.int32 and host.is_contiguous()
    assert np.array_equal(host.numpy(), offsets) and np.array_equal(device.numpy(), offsets)
    assert blocks.shape == (4, 1) and blocks[:, 0].tolist() == [0, 1, 2, 3]


def test_bf16_round_trip_matches_torch():
    rng = np.random.default_rng(1)
    values = np.concatenate([
        rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 4096),
        np.array([0.0, -0.0, np.inf, -np.inf, 1e-40, 3.3895314e38, 1.00390625, 1.01171875], np.float32),
    ]).astype(np.float32)
    ours = oracle.f32_to_bf16(values)
    theirs = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    widened = oracle.bf16_to_f32(ours)
    assert np.array_equal(widened, torch.from_numpy(values).to(torch.bfloat16).float().numpy())


def test_checks_catch_planted_mistakes():
    """Mutants of the oracle, each with one plausible mistake, fail a pinning check."""

    def upper_left(q, k, v, length, scale):
        # Causal mask anchored at key 0 instead of the prefix end.
        out = np.zeros(q.shape)
        tokens = q.shape[2]
        group = q.shape[1] // k.shape[1]
        for hq in range(q.shape[1]):
            for i in range(tokens):
                s = q[0, hq, i] @ k[0, hq // group, : i + 1].T * scale
                w = np.exp(s - s.max())
                out[0, hq, i] = w @ v[0, hq // group, : i + 1] / w.sum()
        return out

    def modulo_heads(q, k, v, length, scale):
        kv_heads = k.shape[1]
        remapped_k = k[:, [hq % kv_heads for hq in range(q.shape[1])]]
        remapped_v = v[:, [hq % kv_heads for hq in range(q.shape[1])]]
        return oracle.flash_attention(q, remapped_k, remapped_v, length, scale)

    def no_scale(q, k, v, length, scale):
        return oracle.flash_attention(q, k, v, length, 1.0)

    def off_by_one(q, k, v, length, scale):
        return oracle.flash_attention(q, k, v, length - 1, scale) if length > q.shape[2] else oracle.flash_attention(q, k, v, length, scale)

    assert not check_kat(upper_left)
    assert not check_gqa_mapping(modulo_heads)
    assert not check_sdpa(no_scale, np.random.default_rng(7))
    assert not check_kat(off_by_one)
