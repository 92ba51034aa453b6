"""torch.export of a step that builds its metadata and calls the batched operators (CPU, fake CUDA).

The reference exporter traces ModelStep.forward, which builds the step's
metadata (compiler/qwen3/model.py:37-47: KVCache -> batched_attention_metadata)
and then runs, per layer, the append and the batched attention
(compiler/qwen3/adapters/attention.py:49-60), with batch in [1, 8] and prefill
tokens in [2, 512] dynamic and backed_size_oblivious set
(compiler/qwen3/export.py:27-56).  Its export tests count one
batched_flash_attention and one append_kv_batched node per layer
(compiler/qwen3/tests/test_export.py:86-169).  The same trace runs here on
fake CUDA tensors, so no GPU is needed.
"""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode
from torch.fx.experimental import _config as symbolic_config

from xinfer_amd.attention import batched_attention_metadata, load_attention_ops

LAYERS = 2


class Step(torch.nn.Module):
    """Metadata once per step, then append + attention per layer, as the adapters order them."""

    def forward(self, q, key, value, positions, kv, kv_lengths, query_lengths):
        offsets, cuda_offsets, blocks = batched_attention_metadata(kv_lengths, query_lengths, q.device)
        out = q.new_zeros(q.shape)
        for layer in range(LAYERS):
            k, v = kv[2 * layer], kv[2 * layer + 1]
            torch.ops.xinfer.append_kv_batched(key, value, positions, cuda_offsets[0], k, v)
            out = out + torch.ops.xinfer.batched_flash_attention(q, k, v, offsets, cuda_offsets, blocks, 128**-0.5)
        return out


@pytest.fixture(scope="module")
def ops(library_path):
    load_attention_ops(library_path)
    return torch.ops.xinfer


def fake_inputs(batch, tokens, capacity=256):
    with FakeTensorMode(allow_non_fake_inputs=True):
        options = dict(dtype=torch.bfloat16, device="cuda")
        q = torch.empty(batch, 16, tokens, 128, **options)
        key = torch.empty(batch, 8, tokens, 128, **options)
        value = torch.empty_like(key)
        positions = torch.empty(batch, tokens, dtype=torch.int64, device="cuda")
        kv = tuple(torch.empty(batch, 8, capacity, 128, **options) for _ in range(2 * LAYERS))
    kv_lengths = torch.tensor([32 + 8 * r for r in range(batch)], dtype=torch.int32)
    query_lengths = torch.tensor([max(1, tokens // (r + 1)) for r in range(batch)], dtype=torch.int32)
    return q, key, value, positions, kv, kv_lengths, query_lengths


@pytest.mark.parametrize("kind", ["prefill", "decode"])
def test_export_batched_step_with_dynamic_batch_and_tokens(ops, kind):
    tokens = 16 if kind == "prefill" else 1
    inputs = fake_inputs(2, tokens)
    batch = torch.export.Dim("batch", min=1, max=8)
    token_shape = {0: batch}
    if kind == "prefill":
        token_shape[2] = torch.export.Dim("tokens", min=2, max=512)
    positions_shape = {0: batch, 1: token_shape[2]} if kind == "prefill" else {0: batch}
    shapes = (token_shape, token_shape, token_shape, positions_shape,
              tuple({0: batch} for _ in range(2 * LAYERS)), {0: batch}, {0: batch})
    with symbolic_config.patch(backed_size_oblivious=True):
        exported = torch.export.export(Step(), inputs, dynamic_shapes=shapes, strict=False)
    targets = [node.target for node in exported.graph.nodes if node.op == "call_function"]
    assert targets.count(ops.batched_flash_attention.default) == LAYERS
    assert targets.count(ops.append_kv_batched.default) == LAYERS
    # The traced metadata copy is a plain device copy (no pinned host tensor).
    assert not any("pin_memory" in str(target) for target in targets)
    symbols = {str(s) for node in exported.graph.nodes if node.op == "placeholder"
               for s in getattr(node.meta.get("val"), "shape", ()) if not isinstance(s, int)}
    assert len(symbols) == (2 if kind == "prefill" else 1), symbols
