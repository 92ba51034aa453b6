"""GPU checks of the native KV append (replacement of compiler/common/kernels/kv_cache.py).

Bit-exact against the CPU oracle append on random bit patterns (NaN/Inf
encodings included), for the vector path (unit feature stride) and the
element path (feature stride 2), with padded positions pointing past the cache
(never dereferenced), out-of-range real positions skipped, the inputs left
unchanged and the cache storage kept in place.
"""

import numpy as np
import pytest
import torch

from attn_helpers import log
from oracle import attention as oracle
from xinfer_amd.kv_cache import append_kv_batched

pytestmark = pytest.mark.gpu


def random_bits(generator, *shape):
    return torch.randint(-(2**15), 2**15, shape, generator=generator, dtype=torch.int32).to(torch.int16)


@pytest.mark.parametrize("feature_stride", [1, 2])
@pytest.mark.parametrize("batch,heads,tokens,dim,capacity", [(1, 8, 512, 128, 4096), (8, 8, 1, 128, 16384),
                                                             (8, 4, 37, 256, 513), (3, 2, 5, 64, 40)])
@torch.inference_mode()
def test_append_matches_oracle(gpu_ops, batch, heads, tokens, dim, capacity, feature_stride):
    generator = torch.Generator().manual_seed(batch * 1000 + tokens + feature_stride)
    log(f"append B={batch} H={heads} T={tokens} D={dim} C={capacity} stride={feature_stride}")
    cache_k = random_bits(generator, batch, heads, capacity, dim)
    cache_v = random_bits(generator, batch, heads, capacity, dim)
    # [B, T, H, D*stride] transposed to [B, H, T, D]: the adapters' layout, optionally strided.
    new_k = random_bits(generator, batch, tokens, heads, dim * feature_stride)
    new_v = random_bits(generator, batch, tokens, heads, dim * feature_stride)
    counts = [tokens if r % 3 == 0 else (0 if r % 3 == 1 else max(1, tokens // 2)) for r in range(batch)]
    positions = torch.full((batch, tokens), capacity + 100, dtype=torch.int64)
    for r, count in enumerate(counts):
        start = int(torch.randint(0, capacity - count + 1, (1,), generator=generator))
        positions[r, :count] = torch.arange(start, start + count)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(counts)]), dtype=torch.int32)
    key_view = new_k[..., ::feature_stride].transpose(1, 2)
    value_view = new_v[..., ::feature_stride].transpose(1, 2)
    expected_k, expected_v = cache_k.numpy().view(np.uint16).copy(), cache_v.numpy().view(np.uint16).copy()
    oracle.append_kv(expected_k, expected_v, key_view.numpy().view(np.uint16), value_view.numpy().view(np.uint16),
                     positions.numpy(), cu.numpy())

    device_k = cache_k.view(torch.bfloat16).cuda()
    device_v = cache_v.view(torch.bfloat16).cuda()
    key = new_k.view(torch.bfloat16).cuda()[..., ::feature_stride].transpose(1, 2)
    value = new_v.view(torch.bfloat16).cuda()[..., ::feature_stride].transpose(1, 2)
    device_positions, device_cu = positions.cuda(), cu.cuda()
    before = [t.clone() for t in (key, value, device_positions, device_cu)]
    pointers = (device_k.data_ptr(), device_v.data_ptr())
    append_kv_batched(key, value, device_positions, device_cu, device_k, device_v)
    assert (device_k.data_ptr(), device_v.data_ptr()) == pointers
    assert torch.equal(device_k.cpu().view(torch.int16), torch.from_numpy(expected_k.view(np.int16)))
    assert torch.equal(device_v.cpu().view(torch.int16), torch.from_numpy(expected_v.view(np.int16)))
    for tensor, original in zip((key, value, device_positions, device_cu), before):
        assert torch.equal(tensor.view(torch.int16) if tensor.dtype == torch.bfloat16 else tensor,
                           original.view(torch.int16) if original.dtype == torch.bfloat16 else original)


@torch.inference_mode()
def test_out_of_range_positions_are_skipped(gpu_ops):
    log("append out-of-range positions")
    cache = torch.zeros(2, 2, 16, 8, dtype=torch.bfloat16, device="cuda")
    other = torch.zeros_like(cache)
    key = torch.ones(2, 2, 3, 8, dtype=torch.bfloat16, device="cuda")
    positions = torch.tensor([[0, 16, -1], [5, 6, 7]], device="cuda")
    cu = torch.tensor([0, 3, 6], dtype=torch.int32, device="cuda")
    append_kv_batched(key, key, positions, cu, cache, other)
    assert cache[0, :, 0].eq(1).all() and cache[1, :, 5:8].eq(1).all()
    assert int(cache.ne(0).sum()) == (1 + 3) * 2 * 8


@torch.inference_mode()
def test_contract_errors(gpu_ops):
    cache = torch.zeros(1, 2, 16, 8, dtype=torch.bfloat16, device="cuda")
    key = torch.ones(1, 2, 3, 8, dtype=torch.bfloat16, device="cuda")
    positions = torch.zeros(1, 3, dtype=torch.int64, device="cuda")
    cu = torch.tensor([0, 3], dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="contiguous"):
        append_kv_batched(key, key, positions, cu, cache.transpose(2, 3), cache.transpose(2, 3))
    with pytest.raises(RuntimeError, match="positions"):
        append_kv_batched(key, key, positions.int(), cu, cache, cache.clone())
