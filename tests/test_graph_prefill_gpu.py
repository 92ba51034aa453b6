"""A prefill (chunked) step captured once in a HIP graph and replayed while the lengths change.

For shapes with more than 8 query vectors per KV head (T * Hq/Hkv > 8),
xinfer::batched_flash_attention_graph plans on the device: a plan kernel
reads every row's query count and KV length from cuda_offsets, picks the key
split size for those lengths, cuts the items into XCD runs of about equal
work, and writes the prefill kernel's and the merge kernel's arguments into
the workspace (prefill.hip: prefill_capture_plan_kernel); the prefill and
merge kernels then read their arguments from there, over grids sized for the
most items the plan can make (blocks past the planned items exit).  Every row
takes the prefill kernel, including rows with one query and rows without
queries (which only zero their outputs).

As for decode (tests/test_graph_decode_gpu.py): the append and the attention
are captured once, and every replay over the length sets below must equal,
bit for bit, the same operators launched eagerly, stay within the float64
oracle's gates, and agree with the default operator (host-planned, other
splits) within the same gates.  Shapes: Qwen3 chunks (G = 2, two query tiles
per row, split rows merged), Qwen3.5 chunks (D = 256, G = 4), eight ragged
Qwen3.5 rows (split and unsplit rows in one launch, cuts inside rows), head
dim 64 with G = 1 (one tile), 64 ragged rows with empty and one-query rows,
and a capacity that needs no split (no merge launch).
"""

import pytest
import torch

from test_graph_decode_gpu import replay_length_sets

pytestmark = pytest.mark.gpu

# (Hq, Hkv, D, T, capacity, length sets: per row (count, length))
SHAPES = {
    "qwen3_chunks": (16, 8, 128, 128, 4096, [
        [(128, 2048), (64, 1000), (1, 300), (0, 5)],
        [(128, 4096), (128, 128), (100, 3000), (2, 2)],
        [(1, 1), (128, 4000), (17, 700), (128, 1024)],
    ]),
    "qwen35_chunks": (16, 4, 256, 64, 2048, [
        [(64, 2048), (1, 77), (33, 1500), (0, 3)],
        [(64, 64), (64, 2000), (2, 2), (64, 1024)],
    ]),
    "qwen35_ragged8": (16, 4, 256, 96, 8192, [
        [(96, 8000), (40, 1200), (96, 3000), (3, 6000), (96, 96), (0, 5), (70, 7000), (1, 1)],
        [(96, 8192), (96, 8100), (1, 4000), (96, 500), (50, 50), (96, 2600), (0, 1), (17, 5000)],
    ]),
    "d64_group1": (8, 8, 64, 40, 1024, [
        [(40, 1024), (5, 500), (40, 40), (1, 1)],
        [(0, 9), (40, 900), (39, 1000), (12, 12)],
    ]),
    # 64 rows: a plan wave lane per row, a whole wave per priced split size.
    "rows64": (16, 8, 64, 16, 2048, [
        [(0 if r % 11 == 4 else (1 if r % 7 == 2 else 16 - r % 5), (r * 2654435761) % 2000 + 16) for r in range(64)],
        [(16 if r % 3 else 5, 2048 if r % 9 == 0 else (r * 40503) % 600 + 16) for r in range(64)],
    ]),
    "no_split": (8, 4, 128, 16, 512, [
        [(16, 512), (1, 1), (16, 16), (0, 2)],
        [(3, 300), (16, 100), (16, 500), (8, 9)],
    ]),
}


@pytest.mark.parametrize("name", list(SHAPES))
@torch.inference_mode()
def test_one_captured_prefill_step_replays_every_length_set(gpu_ops, name):
    replay_length_sets(gpu_ops, name, SHAPES[name])


@torch.inference_mode()
def test_device_counts_beyond_the_capacity_are_clamped(gpu_ops):
    """Device lengths are not validated on the host: a count above the cache
    capacity (here T = 40 queries over C = 32 slots) is taken as min(T, C)
    queries over C keys, and the queries past it are zeroed -- a wrong row,
    never an access outside the tensors."""
    from test_graph_decode_gpu import check_oracle, metadata

    heads, kv_heads, dim, tokens, capacity = 8, 4, 64, 40, 32
    generator = torch.Generator().manual_seed(40)
    q = torch.randn(2, heads, tokens, dim, generator=generator).to(torch.bfloat16).cuda()
    k = torch.randn(2, kv_heads, capacity, dim, generator=generator).to(torch.bfloat16).cuda()
    v = torch.randn(2, kv_heads, capacity, dim, generator=generator).to(torch.bfloat16).cuda()
    host, cu, blocks = metadata([(40, 40), (5, 20)])
    out = gpu_ops.batched_flash_attention_graph(q, k, v, host, cu, blocks, dim**-0.5)
    torch.cuda.synchronize()
    check_oracle(out, q, k, v, [(32, 32), (5, 20)], dim**-0.5)
