"""The committed golden fixtures through the native operators and the C ABI.

Each fixture's K/V prefix is placed in a larger cache whose unused slots --
including, per row, everything past that row's length -- are NaN, and padded
queries are NaN too: the outputs must still match the fixture and padded
queries must come back as exact zeros.
"""

from pathlib import Path

import numpy as np
import pytest
import torch

from attn_helpers import MAX_ABS, MEAN_ABS, log, row_errors
from xinfer_amd.attention import batched_attention_metadata, cache_extent

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "attention_cases.npz"


def load(name):
    with np.load(GOLDEN) as data:
        return {key.split("/")[1]: data[key] for key in data.files if key.startswith(name + "/")}


def names():
    with np.load(GOLDEN) as data:
        return sorted({key.split("/")[0] for key in data.files} - {"append"})


def bits(array):
    return torch.from_numpy(array.view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("name", names())
@torch.inference_mode()
def test_fixture_through_batched_and_flash(gpu_ops, name):
    case = load(name)
    heads, kv_heads, dim, capacity = (int(x) for x in case["geometry"])
    counts, lengths = [int(x) for x in case["counts"]], [int(x) for x in case["lengths"]]
    scale = float(case["scale"])
    batch, tokens, stored = len(counts), max(counts), case["k"].shape[2]
    log(f"golden {name}: counts={counts} lengths={lengths} capacity={capacity}")
    q = bits(case["q"]).cuda()
    k = torch.full((batch, kv_heads, capacity, dim), float("nan"), dtype=torch.bfloat16, device="cuda")
    v = torch.full_like(k, float("nan"))
    k[:, :, :stored] = bits(case["k"]).cuda()
    v[:, :, :stored] = bits(case["v"]).cuda()
    for r, (count, length) in enumerate(zip(counts, lengths)):
        k[r, :, length:] = float("nan")
        v[r, :, length:] = float("nan")
        q[r, :, count:] = float("nan")
    expected = torch.from_numpy(case["expected"])
    host, cu, blocks = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    out = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, scale).cpu()
    for r, count in enumerate(counts):
        assert torch.count_nonzero(out[r, :, count:]).item() == 0
        if count:
            errors = row_errors(out[r, :, :count].float().flatten(1), expected[r, :, :count].flatten(1))
            assert errors["max_abs"] <= MAX_ABS and errors["mean_abs"] <= MEAN_ABS, errors
    if name.startswith("kat"):
        assert torch.equal(out.float(), expected)
    if len(set(lengths)) == 1 and all(c == tokens for c in counts):
        flash = gpu_ops.flash_attention(q, k, v, cache_extent(lengths[0]), scale).cpu()
        assert torch.equal(flash.view(torch.int16), out.view(torch.int16))


@torch.inference_mode()
def test_append_fixture_bit_exact(gpu_ops):
    case = load("append")
    log("golden append")
    cache_k, cache_v = bits(case["cache_k"]).cuda(), bits(case["cache_v"]).cuda()
    gpu_ops.append_kv_batched(bits(case["new_k"]).cuda(), bits(case["new_v"]).cuda(),
                              torch.from_numpy(case["positions"]).cuda(),
                              torch.from_numpy(case["cu_query"]).cuda(), cache_k, cache_v)
    assert torch.equal(cache_k.cpu().view(torch.int16), torch.from_numpy(case["expected_k"].view(np.int16)))
    assert torch.equal(cache_v.cpu().view(torch.int16), torch.from_numpy(case["expected_v"].view(np.int16)))
