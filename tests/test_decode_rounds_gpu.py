"""Decode launches whose items take several rounds of keys.

The planner gives decode items four rounds of keys when one-round items
would number at least 1536 (capi.cpp, make_plan): the block loads and
computes one round at a time, folds the rounds with one rescale each, masks
only the waves whose keys reach the row's end or a query's causal limit, and
writes one output or split record per item.  These cases reach that regime
with rows of one and two queries (the causal limit then differs between a
row's query vectors), rows with no query, lengths that leave the last item
one, two or four rounds long, ending in a partial round, and head dims
padded to 128 and 256.  Keys past each row's length and queries past its count are
NaN, so a read outside them poisons the output.  Each result is checked
against the float64 oracle, and a repeat must be bit-identical.
"""

import numpy as np
import pytest
import torch

from attn_helpers import MAX_ABS, MEAN_ABS, log, row_errors
from oracle import attention as oracle
from xinfer_amd.attention import batched_attention_metadata

pytestmark = pytest.mark.gpu

# (name, Hq, Hkv, D, counts, lengths, capacity).  One-round items per KV head
# and row are ceil(L / keys per round): 256 keys for padded dim 64 and 128 for
# padded dim 128 with up to four query vectors, 32 for padded dim 256 with
# eight.
CASES = (
    # 8 KV heads x (125 + 94 + 71) = 2320 one-round items; rows of two queries.
    ("two_queries_d128", 16, 8, 128, [2, 1, 2, 0], [16000, 12000, 9000, 5], 16384),
    # Head dim 72 (padded to 128); last items of 129, 1 and 385 keys: two
    # rounds, one, and four, each ending in a partial round.
    ("odd_dim_72", 16, 8, 72, [1, 1, 1, 1], [12929, 12801, 12673, 200], 13056),
    # Head dim 200 (padded to 256), GQA group 4 and two queries: 8 query
    # vectors per KV head, the widest decode group (32 keys per round);
    # 4 x (500 + 250 + 65) = 3260 one-round items.
    ("group4_dim200", 16, 4, 200, [2, 1, 1], [16000, 7999, 2049], 16384),
    # Head dim 64: 256 keys per round, no reduce-scatter of the scores;
    # 8 x (25 + 28 + 26 + 36 + 24 + 26 + 27) = 1536 one-round items (the
    # threshold itself), a two-query row, an empty row, partial last rounds.
    ("dim64", 16, 8, 64, [1, 2, 1, 1, 0, 1, 1, 1], [6200, 7000, 6500, 9000, 3, 6144, 6401, 6657], 9216),
    # Head dim 40 (padded to 64), one query vector per KV head (G = 1):
    # 8 x (25 + 26 + 26 + 27 + 24 + 25 + 25 + 26) = 1632 one-round items;
    # the row of 6145 keys ends one key into its last round.
    ("odd_dim_40_g1", 8, 8, 40, [1] * 8, [6400, 6600, 6500, 6700, 6144, 6145, 6300, 6500], 8192),
)


def padded_view(shape, dim, generator):
    """A [.., dim] view of NaN-filled rows 16 elements wider, its first dim features random."""
    wide = torch.full((*shape, dim + 16), float("nan"), dtype=torch.bfloat16)
    wide[..., :dim] = torch.randn(*shape, dim, generator=generator).to(torch.bfloat16)
    return wide.cuda()[..., :dim]


def f64(tensor):
    return tensor.detach().float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("name,heads,kv_heads,dim,counts,lengths,capacity", CASES, ids=[c[0] for c in CASES])
@torch.inference_mode()
def test_multi_round_decode_against_oracle(gpu_ops, name, heads, kv_heads, dim, counts, lengths, capacity):
    batch, tokens = len(counts), max(counts)
    log(f"multi-round decode {name}: Hq={heads} Hkv={kv_heads} D={dim} counts={counts} lengths={lengths} "
        f"C={capacity}")
    generator = torch.Generator().manual_seed(sum(map(ord, name)))
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
    expected = oracle.attention(*(f64(torch.nan_to_num(x, nan=0.0)) for x in (q, k, v)), counts, lengths, scale)
    for r, count in enumerate(counts):
        assert torch.count_nonzero(out[r, :, count:]).item() == 0
        if not count:
            continue
        errors = row_errors(out[r : r + 1, :, :count].float().flatten(1),
                            torch.from_numpy(expected[r : r + 1, :, :count]).float().flatten(1))
        assert errors["max_abs"] <= MAX_ABS and errors["mean_abs"] <= MEAN_ABS, (r, errors)
        assert errors["relative_l2"] < 0.01 and errors["peak_relative"] <= 0.05, (r, errors)
    again = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, scale).cpu()
    assert torch.equal(again.view(torch.int16), out.view(torch.int16))
