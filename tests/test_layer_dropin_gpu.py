"""Whole attention layers: the unmodified transformers modules against the same
layers run through the native operators.

Counterpart of compiler/qwen3/tests/test_attention.py:69-216 and
compiler/qwen35/tests/test_attention.py:25-241.  Each layer is a transformers
module with random weights (no checkpoint).  The reference side runs it
unchanged, with its SDPA attention over an explicit additive mask and a cache
whose update is index_copy_ at the token positions.  The native side restates
the adapters' sequence on the same module's weights
(compiler/qwen3/adapters/attention.py:41-61,
compiler/qwen35/adapters/attention.py:41-64): projections, q/k RMSNorm,
rotary embedding, xinfer::append_kv_batched, xinfer::batched_flash_attention,
the transpose/reshape, the Qwen3.5 output gate and o_proj.  For Qwen3 the fused
variant runs as well: xinfer::qk_norm_rope_append, then
xinfer::batched_flash_attention_bthd.

Checks, as in the reference tests: layer outputs within relative L2 and peak
relative error 0.05 of the transformers module; the caches after the native
append equal the reference caches bit for bit (only the appended slots
change); and the output does not depend on cache contents past each row's
length.  Rows of a ragged batch are compared with the module run row by row.
"""

import pytest
import torch
from torch.nn.attention import SDPBackend, sdpa_kernel

from attn_helpers import log, row_errors
from xinfer_amd.attention import batched_attention_metadata

pytestmark = pytest.mark.gpu

CAPACITY = 16384


class ReferenceCache:
    """The unmodified module's cache: index_copy_ of the new K/V at the token positions.

    The attention modules only call ``update``; transformers' Cache base class
    is not needed for that."""

    def __init__(self, key, value, position):
        self.key, self.value, self.position = key, value, position

    def update(self, key, value, layer_idx, cache_kwargs=None):
        self.key.index_copy_(2, self.position, key)
        self.value.index_copy_(2, self.position, value)
        return self.key, self.value


def reference_row(module, hidden, rotary, key, value, position):
    """One row through the unmodified module: SDPA over the whole cache with the future masked."""
    future = torch.arange(key.shape[2], device="cuda")[None, :] > position[:, None]
    mask = torch.zeros_like(future, dtype=hidden.dtype).masked_fill(future, torch.finfo(hidden.dtype).min)
    cache = ReferenceCache(key, value, position)
    # The memory-efficient kernel, as the reference's Qwen3.5 test pins it: the
    # bf16 MATH path would run batched products on transposed views.
    with sdpa_kernel(SDPBackend.EFFICIENT_ATTENTION):
        return module(hidden, position_embeddings=rotary, attention_mask=mask[None, None],
                      past_key_values=cache)[0]


def native_layer(module, hidden, rotary, key, value, positions, lengths, counts, gated, fused):
    """The adapter's sequence over the native operators, for the whole (ragged) batch."""
    offsets, cuda_offsets, blocks = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    input_shape = hidden.shape[:-1]
    head_shape = (*input_shape, -1, module.head_dim)
    cos, sin = rotary
    if gated:
        from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb

        query, gate = torch.chunk(module.q_proj(hidden).view(*input_shape, -1, module.head_dim * 2), 2, dim=-1)
        gate = gate.reshape(*input_shape, -1)
        q = module.q_norm(query.reshape(head_shape)).transpose(1, 2)
    else:
        from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb

        q = module.q_proj(hidden).view(head_shape)
    k = module.k_proj(hidden).view(head_shape)
    v = module.v_proj(hidden).view(head_shape)
    if fused:
        q = torch.ops.xinfer.qk_norm_rope_append(q, k, v, module.q_norm.weight, module.k_norm.weight,
                                                 module.q_norm.variance_epsilon, cos, sin, positions,
                                                 cuda_offsets[0], key, value)
        out = torch.ops.xinfer.batched_flash_attention_bthd(q, key, value, offsets, cuda_offsets, blocks,
                                                            module.scaling)
        out = out.reshape(*input_shape, -1)
    else:
        if not gated:
            q = module.q_norm(q).transpose(1, 2)
        k = module.k_norm(k).transpose(1, 2)
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        torch.ops.xinfer.append_kv_batched(k, v.transpose(1, 2), positions, cuda_offsets[0], key, value)
        out = torch.ops.xinfer.batched_flash_attention(q, key, value, offsets, cuda_offsets, blocks, module.scaling)
        out = out.transpose(1, 2).reshape(*input_shape, -1).contiguous()
    if gated:
        out = out * torch.sigmoid(gate)
    return module.o_proj(out)


def qwen3_layer():
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Attention, Qwen3Config, Qwen3RotaryEmbedding

    torch.manual_seed(42)
    config = Qwen3Config(hidden_size=1024, intermediate_size=3072, num_hidden_layers=2, num_attention_heads=16,
                         num_key_value_heads=8, head_dim=128, max_position_embeddings=40960, rope_theta=1000000.0,
                         use_sliding_window=False)
    config._attn_implementation = "sdpa"
    module = Qwen3Attention(config, layer_idx=0).eval().requires_grad_(False).to(device="cuda", dtype=torch.bfloat16)
    rotary = Qwen3RotaryEmbedding(config).eval().to("cuda")
    return config, module, lambda hidden, positions: rotary(hidden, positions)


def qwen35_layer():
    from transformers.models.qwen3_5.modeling_qwen3_5 import (Qwen3_5Attention, Qwen3_5TextConfig,
                                                              Qwen3_5TextRotaryEmbedding)

    torch.manual_seed(35)
    config = Qwen3_5TextConfig(hidden_size=1024, num_attention_heads=16, num_key_value_heads=4, head_dim=256,
                               num_hidden_layers=1, layer_types=["full_attention"])
    config._attn_implementation = "sdpa"
    module = Qwen3_5Attention(config, layer_idx=0).eval().requires_grad_(False).to(device="cuda", dtype=torch.bfloat16)
    # The rotary frequencies stay fp32, as in the prepared model; positions are
    # the three identical rows of its multimodal rotary embedding.
    rotary = Qwen3_5TextRotaryEmbedding(config).eval().to("cuda")
    return config, module, lambda hidden, positions: rotary(hidden, positions[None].expand(3, -1, -1))


# (counts, lengths) per row; every row appends its count tokens ending at its length.
QWEN3_CASES = [
    ([1], [1]), ([1], [2]), ([1], [CAPACITY]),
    ([2], [2]), ([2], [3]), ([16], [32]), ([510], [1022]), ([512], [512]), ([512], [CAPACITY]),
    ([1, 1, 1], [5, 700, CAPACITY]), ([16, 1, 0, 200], [40, 3000, 7, 9000]),
]
QWEN35_CASES = [
    ([1], [1]), ([1], [129]), ([2], [3]), ([16], [129]), ([2], [1024]), ([2], [8192]), ([2], [CAPACITY]),
    ([512], [2048]), ([1, 1, 1, 1], [1024, 4096, 8192, CAPACITY]), ([40, 3, 0], [300, 5000, 9]),
]


def run_case(layer, counts, lengths, gated, fused):
    config, module, rotary = layer
    batch, width = len(counts), max(counts)
    kv_heads, dim = config.num_key_value_heads, module.head_dim
    log(f"layer {'qwen3.5' if gated else 'qwen3'}{' fused' if fused else ''}: counts={counts} lengths={lengths}")
    hidden = torch.randn(batch, width, config.hidden_size, device="cuda", dtype=torch.bfloat16)
    positions = torch.stack([torch.arange(n - c, n - c + width, device="cuda") for c, n in zip(counts, lengths)])
    initial = [torch.randn(batch, kv_heads, CAPACITY, dim, device="cuda", dtype=torch.bfloat16) for _ in range(2)]
    # Reference: the unmodified module, row by row over the row's real tokens.
    ref_key, ref_value = (t.clone() for t in initial)
    reference = torch.zeros(batch, width, config.hidden_size, device="cuda", dtype=torch.bfloat16)
    for r, count in enumerate(counts):
        if count:
            reference[r : r + 1, :count] = reference_row(
                module, hidden[r : r + 1, :count], rotary(hidden[r : r + 1, :count], positions[r : r + 1, :count]),
                ref_key[r : r + 1], ref_value[r : r + 1], positions[r, :count])
    key, value = (t.clone() for t in initial)
    pointers = (key.data_ptr(), value.data_ptr())
    actual = native_layer(module, hidden, rotary(hidden, positions), key, value, positions, lengths, counts,
                          gated, fused)
    torch.cuda.synchronize()
    assert (key.data_ptr(), value.data_ptr()) == pointers
    assert bool(torch.isfinite(actual).all())
    for r, count in enumerate(counts):
        if not count:
            continue
        errors = row_errors(actual[r, :count].float(), reference[r, :count].float())
        assert errors["relative_l2"] <= 0.05 and errors["peak_relative"] <= 0.05, (r, errors)
    # Only the appended slots changed.  With the eager norm/RoPE on one full
    # row the projections have the reference's shapes, so the appended rows
    # are the reference module's own bits; otherwise the projection GEMMs run
    # at other shapes (a ragged batch, padded tokens) and may round the last
    # bit differently.
    same_shapes = batch == 1 and counts[0] == width and not fused
    for native, ref, before in ((key, ref_key, initial[0]), (value, ref_value, initial[1])):
        for r, (count, length) in enumerate(zip(counts, lengths)):
            start = length - count
            assert torch.equal(native[r, :, :start], before[r, :, :start])
            assert torch.equal(native[r, :, length:], before[r, :, length:])
            if count:
                appended = row_errors(native[r, :, start:length].float().flatten(1),
                                      ref[r, :, start:length].float().flatten(1))
                assert appended["relative_l2"] <= 0.01, (r, appended)
        if same_shapes:
            assert torch.equal(native, ref)
    # Poisoning every slot past each row's length changes nothing.
    for tensor in (key, value):
        for r, length in enumerate(lengths):
            tensor[r, :, length:] = 100.0
    key_again, value_again = (t.clone() for t in (key, value))
    # Re-append the same tokens (same values), so the step is repeatable.
    again = native_layer(module, hidden, rotary(hidden, positions), key_again, value_again, positions, lengths,
                         counts, gated, fused)
    assert torch.equal(again.view(torch.int16), actual.view(torch.int16))


@pytest.fixture(scope="module")
def qwen3(gpu_ops):
    return qwen3_layer()


@pytest.fixture(scope="module")
def qwen35(gpu_ops):
    return qwen35_layer()


@pytest.mark.parametrize("fused", [False, True], ids=["eager_norm_rope", "fused_norm_rope"])
@pytest.mark.parametrize("counts,lengths", QWEN3_CASES, ids=[f"{c}-{n}" for c, n in QWEN3_CASES])
@torch.inference_mode()
def test_qwen3_layer_matches_transformers(qwen3, counts, lengths, fused):
    run_case(qwen3, counts, lengths, gated=False, fused=fused)


@pytest.mark.parametrize("counts,lengths", QWEN35_CASES, ids=[f"{c}-{n}" for c, n in QWEN35_CASES])
@torch.inference_mode()
def test_qwen35_gated_layer_matches_transformers(qwen35, counts, lengths):
    run_case(qwen35, counts, lengths, gated=True, fused=False)
