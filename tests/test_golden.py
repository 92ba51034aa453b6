"""The committed golden fixtures and the oracle agree (CPU).

tests/golden/make_golden.py wrote the fixtures from the float64 oracle after
checking them against torch's SDPA MATH backend; this test keeps the oracle and
the fixtures from drifting apart and checks the known answers stored in them.
"""

from pathlib import Path

import numpy as np
import pytest

from oracle import attention as oracle

GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_cases.npz"


def cases():
    with np.load(GOLDEN) as data:
        names = sorted({key.split("/")[0] for key in data.files} - {"append"})
    return names


@pytest.mark.parametrize("name", cases())
def test_oracle_reproduces_fixture(name):
    with np.load(GOLDEN) as data:
        case = {key.split("/")[1]: data[key] for key in data.files if key.startswith(name + "/")}
    q, k, v = (oracle.bf16_to_f32(case[x]).astype(np.float64) for x in "qkv")
    out = oracle.attention(q, k, v, case["counts"], case["lengths"], float(case["scale"]))
    np.testing.assert_allclose(out.astype(np.float32), case["expected"], rtol=1e-6, atol=1e-7)
    if name.startswith("kat"):
        assert np.array_equal(case["expected"][0, :, :, 0], np.broadcast_to([1.5, 2.0], case["expected"].shape[1:3]))


def test_append_fixture_is_the_oracle_append():
    with np.load(GOLDEN) as data:
        case = {key.split("/")[1]: data[key] for key in data.files if key.startswith("append/")}
    cache_k, cache_v = case["cache_k"].copy(), case["cache_v"].copy()
    oracle.append_kv(cache_k, cache_v, case["new_k"], case["new_v"], case["positions"], case["cu_query"])
    assert np.array_equal(cache_k, case["expected_k"]) and np.array_equal(cache_v, case["expected_v"])
    # Rows with zero count are untouched; padded positions point outside the cache.
    assert np.array_equal(case["expected_k"][1], case["cache_k"][1])
    assert (case["positions"][1] >= case["cache_k"].shape[2]).all()
