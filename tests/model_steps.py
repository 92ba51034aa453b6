"""Two-layer Qwen3 / Qwen3.5 causal LMs with random weights for the model-step tests.

The configurations are those of the reference's export tests
(compiler/qwen3/tests/test_export.py:62-76: hidden 1024, 16 query / 8 KV heads
of 128, vocabulary 128; compiler/qwen35/tests/test_export.py: 16 / 4 heads of
256, gated full attention).  No checkpoint is read: the weights are
transformers' own initialisation under a fixed seed, with every RMSNorm weight
moved off its initial value so that each norm scales its input.  A model can be
rebuilt from a saved state dict (``build_model(family, state)``), which is how
a fresh process gets the exact weights the packages were compiled with.

Also here: the unmodified transformers model driven row by row, the reference
side of the comparisons (SDPA with an explicit additive causal mask over the
whole cache, and a cache whose update is index_copy_ at the token positions).
"""

import torch

VOCAB, LAYERS, CAPACITY = 128, 2, 1024
# name -> (family, fused norm/rope form)
VARIANTS = {"qwen3": ("qwen3", False), "qwen3_fused": ("qwen3", True), "qwen35": ("qwen35", False)}


def build_model(family, state=None):
    """The bf16 CUDA model of ``family``; random (seeded) weights, or ``state``'s."""
    if family == "qwen3":
        from transformers.models.qwen3.modeling_qwen3 import Qwen3Config, Qwen3ForCausalLM

        config = Qwen3Config(vocab_size=VOCAB, hidden_size=1024, intermediate_size=3072, num_hidden_layers=LAYERS,
                             num_attention_heads=16, num_key_value_heads=8, head_dim=128,
                             max_position_embeddings=CAPACITY, use_sliding_window=False)
        model_class, seed = Qwen3ForCausalLM, 42
    else:
        from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM, Qwen3_5TextConfig

        config = Qwen3_5TextConfig(vocab_size=VOCAB, hidden_size=1024, intermediate_size=3072,
                                   num_hidden_layers=LAYERS, num_attention_heads=16, num_key_value_heads=4,
                                   head_dim=256, layer_types=["full_attention"] * LAYERS,
                                   max_position_embeddings=CAPACITY, tie_word_embeddings=True)
        model_class, seed = Qwen3_5ForCausalLM, 35
    config._attn_implementation = "sdpa"
    torch.manual_seed(seed)
    model = model_class(config).eval().requires_grad_(False)
    if state is None:
        with torch.no_grad():
            for name, parameter in model.named_parameters():
                if name.endswith("norm.weight"):
                    parameter.add_(0.2 * torch.randn_like(parameter))
    else:
        model.load_state_dict(state)
    model = model.to(device="cuda", dtype=torch.bfloat16)
    if family == "qwen35":
        from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5TextRotaryEmbedding

        # The rotary frequencies stay fp32 around the bf16 weights, as in the
        # reference's prepared model (the dtype cast above rounded them).
        model.model.rotary_emb = Qwen3_5TextRotaryEmbedding(config).to("cuda")
    return model


def cache_geometry(model):
    config = model.config
    return config.num_key_value_heads, config.head_dim


class ReferenceCache:
    """The unmodified modules' cache for one row: index_copy_ of the new K/V at the positions."""

    def __init__(self, tensors, position):
        self.tensors, self.position = tensors, position

    def update(self, key, value, layer_idx, cache_kwargs=None):
        k, v = self.tensors[2 * layer_idx], self.tensors[2 * layer_idx + 1]
        k.index_copy_(2, self.position, key)
        v.index_copy_(2, self.position, value)
        return k, v


def transformers_row_logits(model, ids, positions, tensors):
    """Logits of one row's last token through the unmodified model.

    ids/positions [1, n]; tensors: the row's caches (2 per layer, [1, Hkv, C, D]),
    updated in place.  The decoder layers, norm and head are called directly
    with an additive mask that hides every cache slot past each token's
    position; the memory-efficient SDPA kernel, as the reference's tests pin
    it (the bf16 math path would run batched products on transposed views).
    """
    from torch.nn.attention import SDPBackend, sdpa_kernel

    base = model.model
    hidden = base.embed_tokens(ids)
    rotary = base.rotary_emb(hidden, positions)
    capacity = tensors[0].shape[2]
    future = torch.arange(capacity, device=ids.device)[None, :] > positions[0][:, None]
    mask = torch.zeros(future.shape, dtype=hidden.dtype, device=ids.device)
    mask = mask.masked_fill(future, torch.finfo(hidden.dtype).min)[None, None]
    cache = ReferenceCache(tensors, positions[0])
    with sdpa_kernel(SDPBackend.EFFICIENT_ATTENTION):
        for layer in base.layers:
            out = layer(hidden, attention_mask=mask, position_ids=positions, past_key_values=cache,
                        position_embeddings=rotary, use_cache=True)
            hidden = out[0] if isinstance(out, tuple) else out
    return model.lm_head(base.norm(hidden)[:, -1:])[:, 0]


def step_inputs(model, kind, counts, seed, batch_rows=8):
    """(ids, positions, initial caches [batch_rows, ...], kv_lengths, query_lengths, starts) of one case.

    Rows start at position 0 for a 512-token prefill and at 3 + row otherwise
    (compiler/qwen3/tests/test_export.py:113-115); padded tokens repeat the
    row's positions past its count and are never appended.
    """
    generator = torch.Generator(device="cuda").manual_seed(seed)
    batch = len(counts)
    width = max(max(counts), 2 if kind == "prefill" else 1)
    starts = [0 if count == 512 else 3 + row for row, count in enumerate(counts)]
    kv_heads, dim = cache_geometry(model)
    ids = torch.randint(0, VOCAB, (batch, width), device="cuda", generator=generator)
    positions = torch.stack([torch.arange(start, start + width, device="cuda") for start in starts])
    initial = tuple(torch.randn(batch_rows, kv_heads, CAPACITY, dim, device="cuda", generator=generator)
                    .to(torch.bfloat16) for _ in range(2 * LAYERS))
    lengths = torch.tensor([start + count for start, count in zip(starts, counts)], dtype=torch.int32)
    return ids, positions, initial, lengths, torch.tensor(counts, dtype=torch.int32), starts
