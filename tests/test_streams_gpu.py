"""Operators on several streams at once.

The operators enqueue on torch's current stream and take their split-record
workspace from torch's caching allocator on that stream; nothing is shared
between calls (the schedule travels in the kernel arguments).  Two side
streams run a ragged decode batch and a chunked prefill concurrently, several
times over, and every output must equal, bit for bit, the same call made
alone on the default stream.  The KV append runs on a third stream meanwhile
and must leave the same cache contents.
"""

import pytest
import torch

from attn_helpers import log
from xinfer_amd.attention import batched_attention_metadata
from xinfer_amd.workloads import ragged_decode_lengths

pytestmark = pytest.mark.gpu


def inputs(heads, kv_heads, dim, counts, lengths, capacity, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(len(counts), heads, max(counts), dim, generator=g).to(torch.bfloat16).cuda()
    k = torch.randn(len(counts), kv_heads, capacity, dim, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(len(counts), kv_heads, capacity, dim, generator=g).to(torch.bfloat16).cuda()
    host, cu, blocks = batched_attention_metadata(torch.tensor(lengths, dtype=torch.int32),
                                                  torch.tensor(counts, dtype=torch.int32), "cuda")
    return q, k, v, host, cu, blocks, dim ** -0.5


@torch.inference_mode()
def test_concurrent_streams_match_one_stream(gpu_ops):
    decode = inputs(16, 8, 128, [1] * 8, ragged_decode_lengths(0)[0], 16384, seed=1)
    prefill = inputs(16, 8, 128, [512], [2048], 4096, seed=2)
    log("streams: ragged decode and 512-token prefill, alone then on two side streams")
    alone = [gpu_ops.batched_flash_attention(*decode), gpu_ops.batched_flash_attention(*prefill)]

    # The append writes a chunk into its own cache on a third stream.
    g = torch.Generator().manual_seed(3)
    key = torch.randn(2, 8, 64, 128, generator=g).to(torch.bfloat16).cuda()
    value = torch.randn(2, 8, 64, 128, generator=g).to(torch.bfloat16).cuda()
    positions = torch.stack([torch.arange(100, 164), torch.arange(7, 71)]).cuda()
    cu_query = torch.tensor([0, 64, 128], dtype=torch.int32).cuda()
    cache_k = torch.zeros(2, 8, 256, 128, dtype=torch.bfloat16).cuda()
    cache_v = torch.zeros_like(cache_k)
    expect_k, expect_v = cache_k.clone(), cache_v.clone()
    gpu_ops.append_kv_batched(key, value, positions, cu_query, expect_k, expect_v)
    torch.cuda.synchronize()

    streams = [torch.cuda.Stream() for _ in range(3)]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outputs = []
    for _ in range(4):
        with torch.cuda.stream(streams[0]):
            d = gpu_ops.batched_flash_attention(*decode)
        with torch.cuda.stream(streams[1]):
            p = gpu_ops.batched_flash_attention(*prefill)
        with torch.cuda.stream(streams[2]):
            gpu_ops.append_kv_batched(key, value, positions, cu_query, cache_k, cache_v)
        outputs.append((d, p))
    torch.cuda.synchronize()
    for d, p in outputs:
        assert torch.equal(d.view(torch.int16), alone[0].view(torch.int16))
        assert torch.equal(p.view(torch.int16), alone[1].view(torch.int16))
    assert torch.equal(cache_k.view(torch.int16), expect_k.view(torch.int16))
    assert torch.equal(cache_v.view(torch.int16), expect_v.view(torch.int16))
