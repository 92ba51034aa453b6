"""Write the golden attention/append fixtures (tests/golden/attention_cases.npz).

Inputs are seeded bf16 bit patterns; expected outputs come from the float64
oracle (oracle/attention.py) and are cross-checked here against torch's SDPA
MATH backend with the reference tests' lower-right mask before being written.
K/V are stored only up to the longest populated length: tests place them in a
larger cache whose other slots are poisoned, which also checks that nothing
beyond a row's length is read.

    python tests/golden/make_golden.py
"""

from pathlib import Path
import sys

import numpy as np
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import attention as oracle  # noqa: E402

OUTPUT = Path(__file__).resolve().parent / "attention_cases.npz"

# name: (heads, kv_heads, dim, capacity, counts, lengths, kind)
CASES = {
    "kat_16_8_128": (16, 8, 128, 64, [2], [5], "kat"),
    "kat_8_2_256": (8, 2, 256, 64, [2], [5], "kat"),
    "decode_4_2_128": (4, 2, 128, 320, [1, 1], [1, 300], "random"),
    "decode_4_1_256": (4, 1, 256, 300, [1, 1], [257, 64], "random"),
    "decode_multi_query_4_2_128": (4, 2, 128, 220, [2, 4, 3], [200, 5, 150], "random"),
    "prefill_4_2_128": (4, 2, 128, 200, [100], [180], "random"),
    "ragged_4_1_256": (4, 1, 256, 128, [40, 0, 3, 17], [90, 12, 3, 120], "random"),
    "geometry_6_2_64": (6, 2, 64, 160, [16], [129], "random"),
    # Head dims that are not a padded kernel width (the contract is any
    # multiple of 8 in 8..256): a prefill row and two decode rows at D = 72,
    # and a prefill and a decode row with one query head per KV head at D = 136.
    "odd_dim_4_2_72": (4, 2, 72, 160, [30, 1, 2], [120, 77, 2], "random"),
    "odd_dim_3_3_136": (3, 3, 136, 200, [12, 1], [150, 190], "random"),
}
APPEND_CASE = dict(batch=3, heads=2, tokens=6, dim=64, capacity=40, counts=[6, 0, 2])


def bf16_bits(generator, *shape):
    x = torch.randn(*shape, generator=generator, dtype=torch.float32).to(torch.bfloat16)
    return x.view(torch.int16).numpy().view(np.uint16)


def sdpa_check(q, k, v, counts, lengths, scale, expected):
    for r, (count, length) in enumerate(zip(counts, lengths)):
        if not count:
            assert not expected[r].any()
            continue
        mask = torch.arange(length)[None, :] <= torch.arange(length - count, length)[:, None]
        with sdpa_kernel(SDPBackend.MATH):
            ref = F.scaled_dot_product_attention(
                torch.from_numpy(q[r:r + 1, :, :count]),
                torch.from_numpy(k[r:r + 1, :, :length]),
                torch.from_numpy(v[r:r + 1, :, :length]),
                attn_mask=mask, enable_gqa=True, scale=scale,
            ).numpy()
        assert np.allclose(expected[r:r + 1, :, :count], ref, rtol=0, atol=1e-9), "oracle/SDPA disagree"
        assert not expected[r, :, count:].any()


def main():
    arrays = {}
    for seed, (name, (heads, kv_heads, dim, capacity, counts, lengths, kind)) in enumerate(CASES.items()):
        generator = torch.Generator().manual_seed(1000 + seed)
        batch, tokens, stored = len(counts), max(counts), max(lengths)
        if kind == "kat":
            q = np.zeros((batch, heads, tokens, dim), np.uint16)
            k = np.zeros((batch, kv_heads, stored, dim), np.uint16)
            v = oracle.f32_to_bf16(np.broadcast_to(
                np.arange(stored, dtype=np.float32)[None, None, :, None], (batch, kv_heads, stored, dim)))
        else:
            q = bf16_bits(generator, batch, heads, tokens, dim)
            k = bf16_bits(generator, batch, kv_heads, stored, dim)
            v = bf16_bits(generator, batch, kv_heads, stored, dim)
        scale = dim ** -0.5
        qf, kf, vf = (oracle.bf16_to_f32(x).astype(np.float64) for x in (q, k, v))
        expected = oracle.attention(qf, kf, vf, counts, lengths, scale)
        sdpa_check(qf, kf, vf, counts, lengths, scale, expected)
        if kind == "kat":
            assert np.array_equal(expected[0, :, :, 0], np.broadcast_to([1.5, 2.0], (heads, 2)))
        for key, value in dict(q=q, k=k, v=v, counts=np.array(counts, np.int32),
                               lengths=np.array(lengths, np.int32),
                               geometry=np.array([heads, kv_heads, dim, capacity], np.int32),
                               scale=np.array(scale), expected=expected.astype(np.float32)).items():
            arrays[f"{name}/{key}"] = value

    # KV append: random bit patterns (NaN/Inf patterns included) must be copied exactly.
    a = APPEND_CASE
    rng = np.random.default_rng(2024)
    shape_new = (a["batch"], a["heads"], a["tokens"], a["dim"])
    shape_cache = (a["batch"], a["heads"], a["capacity"], a["dim"])
    cache_k = rng.integers(0, 2**16, shape_cache, dtype=np.uint16)
    cache_v = rng.integers(0, 2**16, shape_cache, dtype=np.uint16)
    new_k = rng.integers(0, 2**16, shape_new, dtype=np.uint16)
    new_v = rng.integers(0, 2**16, shape_new, dtype=np.uint16)
    positions = np.full((a["batch"], a["tokens"]), a["capacity"] + 100, np.int64)
    positions[0] = np.arange(30, 36)
    positions[2, :2] = [0, 39]
    cu = np.concatenate([[0], np.cumsum(a["counts"])]).astype(np.int32)
    expected_k, expected_v = cache_k.copy(), cache_v.copy()
    oracle.append_kv(expected_k, expected_v, new_k, new_v, positions, cu)
    for key, value in dict(cache_k=cache_k, cache_v=cache_v, new_k=new_k, new_v=new_v,
                           positions=positions, cu_query=cu, expected_k=expected_k,
                           expected_v=expected_v).items():
        arrays[f"append/{key}"] = value

    np.savez_compressed(OUTPUT, **arrays)
    print(f"wrote {OUTPUT} ({OUTPUT.stat().st_size} bytes, {len(CASES)} attention cases + append)")


if __name__ == "__main__":
    main()
