"""A decode step captured once in a HIP graph and replayed while the lengths change.

xinfer::batched_flash_attention_graph (C ABI xinfer_batched_flash_attention_graph)
reads each row's query count and KV length from cuda_offsets when its kernels
run, so one captured step -- the native append, then the attention -- serves
every length set.  Between replays the test rewrites the device metadata, the
positions, the new tokens and the queries in place (the serving loop's
per-step writes), runs other eager work and synchronises; every replay must
equal, bit for bit, the same two operators launched eagerly on a copy of the
caches, and stay within the oracle gates.  The default operator, whose plan
comes from host lengths, agrees within the same gates.

Launch shapes covered (capi.cpp, check_capture): the Qwen3 and Qwen3.5
decode shapes and the head-dim-64 shape take four-round items, one block
each; the two-token shapes take one-round items with one block per item; the
64-row batch at capacity 16384 has 65536 one-round items in a grid capped at
2048 blocks, so every block takes several items in turn (blockIdx.x,
blockIdx.x + 2048, ...) and reuses its reduction buffers between them.  Query
vectors per KV head: 2 (Qwen3), 4 (Qwen3.5, two tokens), 1 (head dim 64,
G = 1) and 8 (two tokens with G = 4).
"""

import numpy as np
import pytest
import torch

from attn_helpers import MAX_ABS, MEAN_ABS, log, row_errors
from oracle import attention as oracle
from xinfer_amd.attention import batched_attention_metadata

pytestmark = pytest.mark.gpu

# (Hq, Hkv, D, T, capacity, length sets: per row (count, length))
SHAPES = {
    "qwen3_decode": (16, 8, 128, 1, 16384, [
        [(1, 13312), (1, 2162), (1, 386), (1, 9459), (1, 1399), (1, 3852), (1, 55), (1, 182)],
        [(1, 24), (1, 75), (1, 81), (1, 54), (1, 755), (1, 34), (1, 390), (1, 2170)],
        [(1, 16384), (0, 7), (1, 1), (1, 129), (1, 128), (1, 127), (0, 1), (1, 16000)],
        [(1, 5), (1, 5), (1, 5), (1, 5), (1, 5), (1, 5), (1, 5), (1, 5)],
    ]),
    "qwen35_decode": (16, 4, 256, 1, 16384, [
        [(1, 1024), (1, 4096), (1, 8192), (1, 16384)],
        [(1, 3), (0, 9), (1, 700), (1, 65)],
        [(1, 16384), (1, 16384), (1, 1), (1, 2)],
    ]),
    "two_tokens": (8, 4, 128, 2, 4096, [
        [(2, 300), (1, 4096), (0, 5), (2, 2)],
        [(1, 1), (2, 3000), (2, 129), (1, 700)],
    ]),
    # G = 4 and two tokens: eight query vectors per KV head.
    "two_tokens_group4": (16, 4, 128, 2, 4096, [
        [(2, 4096), (1, 77), (2, 1500), (0, 3)],
        [(2, 2), (2, 4000), (1, 1), (2, 640)],
    ]),
    # Head dim 64, G = 1: 256 keys per round, four-round items.
    "d64_group1": (8, 8, 64, 1, 8192, [
        [(1, 8192), (1, 5000), (1, 1), (1, 257), (0, 9), (1, 1024), (1, 3333), (1, 7777)],
        [(1, 3), (1, 8191), (1, 600), (1, 6000), (1, 2), (1, 4097), (0, 1), (1, 1025)],
    ]),
    # 64 rows at capacity 16384: a grid capped at 2048 blocks over up to
    # 65536 items, with ragged and empty rows.
    "capped_grid_b64": (16, 8, 128, 1, 16384, [
        [(0 if r % 13 == 5 else 1, (r * 2654435761) % 16384 + 1) for r in range(64)],
        [(0 if r % 7 == 3 else 1, 16384 if r % 9 == 0 else (r * 40503) % 3000 + 1) for r in range(64)],
    ]),
}


def metadata(rows):
    counts = torch.tensor([c for c, _ in rows], dtype=torch.int32)
    lengths = torch.tensor([n for _, n in rows], dtype=torch.int32)
    return batched_attention_metadata(lengths, counts, "cuda")


def check_oracle(out, q, k, v, rows, scale):
    """Each row against the float64 oracle over its own populated prefix only."""
    out = out.cpu()
    for r, (count, length) in enumerate(rows):
        assert torch.count_nonzero(out[r, :, count:]).item() == 0
        if count:
            expected = oracle.attention(*(x[r : r + 1, :, :n].float().cpu().numpy().astype(np.float64)
                                          for x, n in ((q, count), (k, length), (v, length))),
                                        [count], [length], scale)
            errors = row_errors(out[r, :, :count].float().flatten(1),
                                torch.from_numpy(expected[0]).float().flatten(1))
            assert errors["max_abs"] <= MAX_ABS and errors["mean_abs"] <= MEAN_ABS, (r, errors)


def replay_length_sets(gpu_ops, name, shape):
    """Capture append + graph attention once for `shape`, then replay it over
    every length set twice, each replay checked against the eager operators,
    the float64 oracle and the default operator."""
    heads, kv_heads, dim, tokens, capacity, length_sets = shape
    batch = len(length_sets[0])
    scale = dim**-0.5
    generator = torch.Generator().manual_seed(sum(map(ord, name)))
    options = dict(device="cuda", dtype=torch.bfloat16)

    def draw(*shape):
        return torch.randn(*shape, generator=generator).to(torch.bfloat16).cuda()

    # Static inputs of the captured step, rewritten in place before each replay.
    q = torch.empty(batch, heads, tokens, dim, **options)
    new_k = torch.empty(batch, kv_heads, tokens, dim, **options)
    new_v = torch.empty_like(new_k)
    positions = torch.empty(batch, tokens, dtype=torch.int64, device="cuda")
    k, v = draw(batch, kv_heads, capacity, dim), draw(batch, kv_heads, capacity, dim)
    host, cu, blocks = metadata(length_sets[0])

    def set_step(rows):
        q.copy_(draw(batch, heads, tokens, dim))
        new_k.copy_(draw(batch, kv_heads, tokens, dim))
        new_v.copy_(draw(batch, kv_heads, tokens, dim))
        step_positions = torch.full((batch, tokens), capacity + 100, dtype=torch.int64)
        for r, (count, length) in enumerate(rows):
            step_positions[r, :count] = torch.arange(length - count, length)
        positions.copy_(step_positions)
        step_host, step_cu, _ = metadata(rows)
        cu.copy_(step_cu)
        host.copy_(step_host)
        return step_host, step_cu

    def step(kk, vv, host_offsets, cuda_offsets):
        gpu_ops.append_kv_batched(new_k, new_v, positions, cuda_offsets[0], kk, vv)
        return gpu_ops.batched_flash_attention_graph(q, kk, vv, host_offsets, cuda_offsets, blocks, scale)

    # Warm up on a side stream, then capture once.
    set_step(length_sets[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(k.clone(), v.clone(), host, cu)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step(k, v, host, cu)
    torch.cuda.synchronize()

    for round_ in range(2):
        for rows in length_sets:
            log(f"graph step {name} round {round_}: rows={rows}")
            set_step(rows)
            k_before, v_before = k.clone(), v.clone()
            torch.cuda.synchronize()
            graph.replay()
            # Other eager work between the replay and the checks.
            _ = torch.randn(1 << 20, device="cuda").sum()
            torch.cuda.synchronize()
            k_eager, v_eager = k_before.clone(), v_before.clone()
            eager = step(k_eager, v_eager, host, cu)
            torch.cuda.synchronize()
            assert torch.equal(captured.view(torch.int16), eager.view(torch.int16))
            assert torch.equal(k.view(torch.int16), k_eager.view(torch.int16))
            assert torch.equal(v.view(torch.int16), v_eager.view(torch.int16))
            check_oracle(captured, q, k, v, rows, scale)
            default = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, scale)
            torch.cuda.synchronize()
            delta = (default.float() - captured.float()).abs()
            assert float(delta.max()) <= MAX_ABS and float(delta.mean()) <= MEAN_ABS


@pytest.mark.parametrize("name", list(SHAPES))
@torch.inference_mode()
def test_one_captured_step_replays_every_length_set(gpu_ops, name):
    replay_length_sets(gpu_ops, name, SHAPES[name])


@torch.inference_mode()
def test_graph_mode_rejects_more_than_64_rows(gpu_ops):
    q = torch.zeros(65, 16, 1, 128, device="cuda", dtype=torch.bfloat16)
    k = torch.zeros(65, 8, 256, 128, device="cuda", dtype=torch.bfloat16)
    host, cu, blocks = metadata([(1, 32)] * 65)
    with pytest.raises(RuntimeError, match="Graph-capture attention takes at most 64 rows"):
        gpu_ops.batched_flash_attention_graph(q, k, k, host, cu, blocks, 128**-0.5)
