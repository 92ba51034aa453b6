"""Head dims other than 64 / 128 / 256 through every kernel path.

The reference accepts any head dim that is a multiple of 8 in 8..256
(compiler/common/kernels/attention.cpp:96-97).  The kernels here are built for
padded dims 64, 128 and 256; a smaller D runs the next padded kernel, whose
lanes past D must neither read past a key row's D features nor write past
the output row's.  Each case checks against the float64 oracle:

* decode rows (G * count <= 8 query vectors per KV head) with one item, with
  a few splits (the one-thread-per-vector merge), with many splits (the
  split-lane merge) and with more than 64 (the feature-sliced merge);
* prefill rows with and without key splits, and a row with G = 1;
* K/V/Q stored as views of wider rows whose gap holds NaN, so a read past D
  poisons the output.
"""

import numpy as np
import pytest
import torch

from attn_helpers import MAX_ABS, MEAN_ABS, log, row_errors
from oracle import attention as oracle
from xinfer_amd.attention import batched_attention_metadata

pytestmark = pytest.mark.gpu

DIMS = (8, 32, 72, 96, 136, 192, 248)

# (name, Hq, Hkv, counts, lengths, capacity)
CASES = (
    ("decode_one_item", 8, 4, [1, 1, 1], [1, 37, 100], 128),
    ("decode_few_splits", 8, 4, [1, 2, 1], [700, 300, 1], 1024),
    ("decode_many_splits", 8, 4, [1, 1], [3000, 57], 3072),
    # Past 64 splits the merge cuts a vector's features into blocks of 64
    # (and past 256 splits, 512-thread blocks): 258 splits at padded dims 256
    # (two-round items) and 128, 129 at 64.
    ("decode_sliced_merge", 8, 4, [1, 1], [33000, 70], 33024),
    ("decode_group1", 4, 4, [1, 4], [900, 200], 1024),
    ("prefill_unsplit", 8, 4, [100, 1], [300, 64], 512),
    ("prefill_split", 8, 4, [200, 64, 0], [2100, 1500, 9], 2176),
    ("prefill_group1", 4, 4, [40, 3], [1200, 40], 1280),
)


def padded_view(shape, dim, generator):
    """A [.., dim] view of NaN-filled rows 16 elements wider, its first dim features random."""
    wide = torch.full((*shape, dim + 16), float("nan"), dtype=torch.bfloat16)
    wide[..., :dim] = torch.randn(*shape, dim, generator=generator).to(torch.bfloat16)
    return wide.cuda()[..., :dim]


def f64(tensor):
    return tensor.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("dim", DIMS)
@pytest.mark.parametrize("name,heads,kv_heads,counts,lengths,capacity", CASES, ids=[c[0] for c in CASES])
@torch.inference_mode()
def test_head_dim_against_oracle(gpu_ops, dim, name, heads, kv_heads, counts, lengths, capacity):
    batch, tokens = len(counts), max(max(counts), 1)
    log(f"head dim {dim} {name}: Hq={heads} Hkv={kv_heads} counts={counts} lengths={lengths} C={capacity}")
    generator = torch.Generator().manual_seed(dim * 1000 + len(name))
    q = padded_view((batch, heads, tokens), dim, generator)
    k = padded_view((batch, kv_heads, capacity), dim, generator)
    v = padded_view((batch, kv_heads, capacity), dim, generator)
    for r, (count, length) in enumerate(zip(counts, lengths)):
        k[r, :, length:] = float("nan")
        v[r, :, length:] = float("nan")
        q[r, :, count:] = float("nan")
    host, cu, blocks = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    scale = dim ** -0.5
    out = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, scale)
    torch.cuda.synchronize()
    out = out.cpu()
    assert out.is_contiguous() and out.shape == (batch, heads, tokens, dim)
    q_valid = torch.nan_to_num(q, nan=0.0)
    k_valid = torch.nan_to_num(k, nan=0.0)
    v_valid = torch.nan_to_num(v, nan=0.0)
    expected = oracle.attention(f64(q_valid), f64(k_valid), f64(v_valid), counts, lengths, scale)
    for r, count in enumerate(counts):
        assert torch.count_nonzero(out[r, :, count:]).item() == 0
        if not count:
            continue
        actual = out[r : r + 1, :, :count].float().flatten(1)
        reference = torch.from_numpy(expected[r : r + 1, :, :count]).float().flatten(1)
        errors = row_errors(actual, reference)
        assert errors["max_abs"] <= MAX_ABS and errors["mean_abs"] <= MEAN_ABS, errors
        assert errors["relative_l2"] < 0.01 and errors["peak_relative"] <= 0.05, errors
    # The schedule depends only on the lengths: a repeat is bit-identical.
    again = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, scale).cpu()
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))
