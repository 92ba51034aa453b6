"""The page table of xinfer::batched_flash_attention: the `blocks` argument.

The reference hands `blocks` [B, 1] to its paged FlashAttention call whenever
the cache capacity is a multiple of 256 (compiler/common/kernels/attention.cpp:
39-40, 56-58, 68-70): row r then reads its keys and values from cache row
blocks[r], and for other capacities the table is ignored.  The kernels read
the table on the device (each work item issues its first K/V loads for row r
and reloads them only when the page differs).

Each case runs the operator with a page table that is not the identity and
compares, bit for bit, with the identity table over caches whose rows were
copied to where the table points (k_moved[r] = k[blocks[r]]); the moved run
must also pass the float64 oracle's gates.  Cache rows that no row's page
names are NaN, so a read of the wrong row poisons the output.  Tables: a
permutation, a repeating table, entries out of [0, B) (clamped into it), and
a table viewed with a row stride of 2.  Paths: one-round and four-round
decode, decode rows merged inside the decode launch, prefill at head dims
128 and 256 with and without key splits, head dim 64, the [B, T, Hq, D]
output and the capture-once operator (decode and prefill shapes).  A
capacity that is not a multiple of 256 ignores the table.
"""

import numpy as np
import pytest
import torch

from attn_helpers import MAX_ABS, MEAN_ABS, log, row_errors
from oracle import attention as oracle
from xinfer_amd.attention import batched_attention_metadata

pytestmark = pytest.mark.gpu

# (name, Hq, Hkv, D, counts, lengths, capacity)
CASES = (
    ("decode_one_round", 16, 8, 128, [1, 1, 0, 1], [300, 5, 3, 1000], 1024),
    ("decode_four_rounds", 16, 8, 128, [1, 1, 1, 1, 1, 1, 1, 1],
     [3000, 2900, 3100, 2500, 3500, 2800, 3300, 3200], 4096),  # 1544 one-round items: four rounds
    ("decode_merged_in_launch", 16, 8, 128, [1, 1], [1024, 900], 2048),
    ("decode_dim256", 16, 4, 256, [1, 1, 1], [4000, 100, 2048], 4096),
    ("prefill_dim128", 16, 8, 128, [100, 37, 64], [600, 37, 2000], 2048),
    ("prefill_dim256", 16, 4, 256, [60, 130], [500, 1300], 1536),
    ("mixed_dim64", 8, 4, 64, [1, 40, 1], [500, 300, 20], 512),
)


def tables(batch):
    """Non-identity page tables of a batch: (name, entries as given, entries after clamping)."""
    perm = [(r + 1) % batch for r in range(batch)]
    repeat = [min(batch - 1, 2 * (r // 2) + 1) for r in range(batch)]
    wild = [-5 if r % 2 else batch + 3 for r in range(batch)]
    return (("permutation", perm, perm), ("repeating", repeat, repeat),
            ("out_of_range", wild, [0 if r % 2 else batch - 1 for r in range(batch)]))


def device_table(entries, stride2=False):
    """[B, 1] int32 CUDA table; with stride2, a column view of a [B, 2] tensor (row stride 2)."""
    column = torch.tensor(entries, dtype=torch.int32).view(-1, 1)
    if stride2:
        return torch.cat((column, torch.full_like(column, 12345)), dim=1).cuda()[:, :1]
    return column.cuda()


def make_inputs(name, heads, kv_heads, dim, counts, lengths, capacity, pages):
    """Seeded inputs; cache rows no page names are NaN, and so is every key past
    the longest length of the rows that read a cache row."""
    generator = torch.Generator().manual_seed(sum(map(ord, name)))
    batch, tokens = len(counts), max(max(counts), 1)
    q = torch.randn(batch, heads, tokens, dim, generator=generator).to(torch.bfloat16)
    k = torch.randn(batch, kv_heads, capacity, dim, generator=generator).to(torch.bfloat16)
    v = torch.randn(batch, kv_heads, capacity, dim, generator=generator).to(torch.bfloat16)
    for r, count in enumerate(counts):
        q[r, :, count:] = float("nan")
    for row in range(batch):
        readers = [lengths[r] for r in range(batch) if pages[r] == row]
        end = max(readers) if readers else 0
        k[row, :, end:] = float("nan")
        v[row, :, end:] = float("nan")
    return q.cuda(), k.cuda(), v.cuda()


def f64(tensor):
    return tensor.detach().float().cpu().numpy().astype(np.float64)


def bits(tensor):
    return tensor.contiguous().view(torch.int16)


@pytest.mark.parametrize("name,heads,kv_heads,dim,counts,lengths,capacity", CASES, ids=[c[0] for c in CASES])
@torch.inference_mode()
def test_page_table_reads_the_named_rows(gpu_ops, name, heads, kv_heads, dim, counts, lengths, capacity):
    batch = len(counts)
    host, cu, identity = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    scale = dim ** -0.5
    for table, entries, pages in tables(batch):
        for stride2 in (False, True):
            log(f"page table {name} {table} stride={2 if stride2 else 1}: counts={counts} lengths={lengths} "
                f"C={capacity} pages={pages}")
            q, k, v = make_inputs(name, heads, kv_heads, dim, counts, lengths, capacity, pages)
            blocks = device_table(entries, stride2)
            assert blocks.stride(0) == (2 if stride2 else 1)
            out = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, scale)
            moved_k, moved_v = k[pages].contiguous(), v[pages].contiguous()
            expected = gpu_ops.batched_flash_attention(q, moved_k, moved_v, host, cu, identity, scale)
            torch.cuda.synchronize()
            assert torch.equal(bits(out), bits(expected)), (name, table, stride2)
            bthd = gpu_ops.batched_flash_attention_bthd(q, k, v, host, cu, blocks, scale)
            torch.cuda.synchronize()
            assert torch.equal(bits(bthd.transpose(1, 2)), bits(out)), (name, table, stride2)
        reference = oracle.attention(*(f64(torch.nan_to_num(x, nan=0.0)) for x in (q, moved_k, moved_v)),
                                     counts, lengths, scale)
        result = out.float().cpu()
        for r, count in enumerate(counts):
            assert torch.count_nonzero(result[r, :, count:]).item() == 0
            if not count:
                continue
            errors = row_errors(result[r : r + 1, :, :count].flatten(1),
                                torch.from_numpy(reference[r : r + 1, :, :count]).float().flatten(1))
            assert errors["max_abs"] <= MAX_ABS and errors["mean_abs"] <= MEAN_ABS, (name, table, r, errors)
            assert errors["relative_l2"] < 0.01 and errors["peak_relative"] <= 0.05, (name, table, r, errors)


# (name, Hq, Hkv, D, counts, lengths, capacity) of the capture-once operator:
# decode kernels, and the device-planned prefill kernels (split and unsplit rows).
CAPTURE_CASES = (
    ("capture_decode", 16, 8, 128, [1, 1, 1, 0], [700, 1500, 33, 9], 2048),
    ("capture_prefill_dim128", 16, 8, 128, [100, 1, 64, 0], [2000, 33, 64, 9], 2048),
    ("capture_prefill_dim256", 16, 4, 256, [60, 130, 7], [1500, 1300, 7], 1536),
)


@pytest.mark.parametrize("name,heads,kv_heads,dim,counts,lengths,capacity", CAPTURE_CASES,
                         ids=[c[0] for c in CAPTURE_CASES])
@torch.inference_mode()
def test_capture_operator_reads_the_named_rows(gpu_ops, name, heads, kv_heads, dim, counts, lengths, capacity):
    """The capture-once operator reads the table on the device too."""
    host, cu, identity = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    for table, entries, pages in tables(len(counts)):
        log(f"{name}, page table {table}: counts={counts} lengths={lengths} pages={pages}")
        q, k, v = make_inputs(name, heads, kv_heads, dim, counts, lengths, capacity, pages)
        out = gpu_ops.batched_flash_attention_graph(q, k, v, host, cu, device_table(entries), dim ** -0.5)
        expected = gpu_ops.batched_flash_attention_graph(q, k[pages].contiguous(), v[pages].contiguous(), host, cu,
                                                         identity, dim ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(expected)), table
        assert not bool(torch.isnan(out.float()).any()), table


@torch.inference_mode()
def test_capacity_not_a_multiple_of_256_ignores_the_table(gpu_ops):
    """As in the reference, whose unpaged path packs k[r]/v[r] (attention.cpp:47-51)."""
    counts, lengths, capacity = [1, 30, 1], [700, 500, 9], 1000
    host, cu, identity = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    generator = torch.Generator().manual_seed(7)
    q = torch.randn(3, 16, 30, 128, generator=generator).to(torch.bfloat16).cuda()
    k = torch.randn(3, 8, capacity, 128, generator=generator).to(torch.bfloat16).cuda()
    v = torch.randn(3, 8, capacity, 128, generator=generator).to(torch.bfloat16).cuda()
    expected = gpu_ops.batched_flash_attention(q, k, v, host, cu, identity, 128 ** -0.5)
    for _, entries, _ in tables(3):
        out = gpu_ops.batched_flash_attention(q, k, v, host, cu, device_table(entries), 128 ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(bits(out), bits(expected))
