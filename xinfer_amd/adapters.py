"""Model-side callers of the attention operators.

transformers attention modules rewired to the native operators, and an
explicit inference step that drives unchanged transformers decoder layers with
caller-owned KV tensors, so that a whole model step exports (torch.export) and
packages (``package.compile_package``) with one append and one batched
attention call per layer.  Counterparts of the reference's adapters and steps:

* Qwen3: compiler/qwen3/adapters/attention.py:10-68 (the adapter and its
  installation) and compiler/qwen3/model.py:37-95 (KVCache, ModelStep);
* Qwen3.5 full-attention layers: compiler/qwen35/adapters/attention.py:10-76
  and compiler/qwen35/model.py:144-183.  The Qwen3.5 linear-attention (Gated
  DeltaNet) layers and their recurrent state are not attention operators and
  are not part of this library: ``ModelStep`` accepts models whose layers are
  all full attention.

Besides the reference's sequence (projections, q/k RMSNorm, rotary embedding,
``append_kv_batched``, ``batched_flash_attention``, transpose, o_proj), the
Qwen3 adapter has a fused form: ``qk_norm_rope_append`` (RMSNorm, rotary
embedding and append in one native launch) followed by
``batched_flash_attention_bthd``, whose [B, T, Hq, D] output makes the
reshape before o_proj a view.

The adapters reject what the native path does not implement, with ValueError
as the reference's adapters do: training mode, returned attention weights, an
explicit attention mask (causality comes from the cache lengths), a cache that
is not this module's KVCache, and a position tensor other than the cache's.
"""

from __future__ import annotations

import torch

from .attention import batched_attention_metadata, load_attention_ops, require

# Export bounds of the model steps (compiler/qwen35/config.py:8-9): batch and
# prefill tokens per step.
MAX_PREFILL = 512
MAX_BATCH_SIZE = 8


class KVCache:
    """Caller-owned KV tensors of one step, with its positions and attention metadata.

    ``tensors[2 * i]`` and ``tensors[2 * i + 1]`` are layer i's key and value
    caches, contiguous bf16 [B, Hkv, C, D]; ``position`` holds the step's token
    positions [B, T] (int64, on the device); ``kv_lengths`` and
    ``query_lengths`` are CPU int32 [B]: each row's populated length after the
    step and its real new tokens.  The metadata is built once per step and
    shared by every layer.  ``update`` is the call transformers attention
    modules make on their cache: it appends in place and returns the layer's
    whole caches, whose rows the attention reads up to each row's length.
    """

    def __init__(self, tensors, position, kv_lengths, query_lengths):
        self.tensors = tuple(tensors)
        self.position = position
        self.offsets, self.cuda_offsets, self.blocks = batched_attention_metadata(
            kv_lengths, query_lengths, position.device
        )

    def layer(self, index):
        return self.tensors[2 * index], self.tensors[2 * index + 1]

    def update(self, key, value, layer_idx, cache_kwargs=None):
        """Append key/value [B, Hkv, T, D] at the step's positions (real tokens only)."""
        cache_key, cache_value = self.layer(layer_idx)
        torch.ops.xinfer.append_kv_batched(key, value, self.position, self.cuda_offsets[0], cache_key, cache_value)
        return cache_key, cache_value


def _check_geometry(module):
    config = module.config
    heads, kv_heads, dim = config.num_attention_heads, config.num_key_value_heads, module.head_dim
    require(heads > 0 and kv_heads > 0 and heads % kv_heads == 0, "Query heads must be a positive multiple of KV heads")
    require(8 <= dim <= 256 and dim % 8 == 0, "Flash head dimension must be a multiple of 8 in 8..256")


def _step_cache(adapter, attention_mask, kwargs):
    """The call's KVCache, after the checks every adapter makes."""
    require(not adapter.training and not kwargs.get("output_attentions", False),
            "Flash adapter supports inference without attention weights")
    require(attention_mask is None, "Flash adapter uses KVCache lengths instead of attention masks")
    cache = kwargs.get("past_key_values")
    if cache is None:
        cache = kwargs.get("past_key_value")
    require(isinstance(cache, KVCache), "Flash adapter requires a KVCache with per-row lengths")
    position = kwargs.get("cache_position")
    require(position is None or position is cache.position, "Flash adapter requires KVCache with the same position tensor")
    return cache


class Qwen3FlashAttention(torch.nn.Module):
    """Qwen3Attention's weights and arithmetic around the native operators.

    ``fused=False`` is the reference adapter's sequence; ``fused=True`` runs
    the q/k RMSNorm, the rotary embedding and the append as one
    ``qk_norm_rope_append`` launch (same bf16 rounding points) and takes the
    attention output in [B, T, Hq, D].
    """

    def __init__(self, original, *, fused=False):
        super().__init__()
        from transformers.models.qwen3.modeling_qwen3 import Qwen3Attention

        require(type(original) is Qwen3Attention and original.sliding_window is None,
                "Expected full-attention Qwen3Attention")
        _check_geometry(original)
        if fused:
            require(original.q_norm.variance_epsilon == original.k_norm.variance_epsilon,
                    "The fused norm/rope step needs one RMSNorm epsilon for q and k")
        self.original = original
        self.fused = fused

    def forward(self, hidden_states, position_embeddings, attention_mask=None, **kwargs):
        from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb

        cache = _step_cache(self, attention_mask, kwargs)
        a = self.original
        batch_shape = hidden_states.shape[:-1]
        per_head = (*batch_shape, -1, a.head_dim)
        cos, sin = position_embeddings
        key_cache, value_cache = cache.layer(a.layer_idx)
        if self.fused:
            q = a.q_proj(hidden_states).view(per_head)
            k = a.k_proj(hidden_states).view(per_head)
            v = a.v_proj(hidden_states).view(per_head)
            q = torch.ops.xinfer.qk_norm_rope_append(q, k, v, a.q_norm.weight, a.k_norm.weight,
                                                     a.q_norm.variance_epsilon, cos, sin, cache.position,
                                                     cache.cuda_offsets[0], key_cache, value_cache)
            out = torch.ops.xinfer.batched_flash_attention_bthd(q, key_cache, value_cache, cache.offsets,
                                                                cache.cuda_offsets, cache.blocks, a.scaling)
            return a.o_proj(out.reshape(*batch_shape, -1)), None
        q = a.q_norm(a.q_proj(hidden_states).view(per_head)).transpose(1, 2)
        k = a.k_norm(a.k_proj(hidden_states).view(per_head)).transpose(1, 2)
        v = a.v_proj(hidden_states).view(per_head).transpose(1, 2)
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        key_cache, value_cache = cache.update(k, v, a.layer_idx)
        out = torch.ops.xinfer.batched_flash_attention(q, key_cache, value_cache, cache.offsets, cache.cuda_offsets,
                                                       cache.blocks, a.scaling)
        return a.o_proj(out.transpose(1, 2).reshape(*batch_shape, -1).contiguous()), None


class Qwen35FlashAttention(torch.nn.Module):
    """Qwen3.5's gated full attention around the native operators.

    q_proj yields the query and a per-feature output gate; the attention
    output is multiplied by sigmoid(gate) before o_proj.  The rotary
    embedding covers the first rotary_dim features of each head (partial
    rotary), which apply_rotary_pos_emb handles.
    """

    def __init__(self, original):
        super().__init__()
        from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5Attention

        require(type(original) is Qwen3_5Attention, "Expected Qwen3.5 full attention")
        _check_geometry(original)
        self.original = original

    def forward(self, hidden_states, position_embeddings, attention_mask=None, **kwargs):
        from transformers.models.qwen3_5.modeling_qwen3_5 import apply_rotary_pos_emb

        cache = _step_cache(self, attention_mask, kwargs)
        a = self.original
        batch_shape = hidden_states.shape[:-1]
        per_head = (*batch_shape, -1, a.head_dim)
        query, gate = torch.chunk(a.q_proj(hidden_states).view(*batch_shape, -1, 2 * a.head_dim), 2, dim=-1)
        gate = gate.reshape(*batch_shape, -1)
        q = a.q_norm(query.reshape(per_head)).transpose(1, 2)
        k = a.k_norm(a.k_proj(hidden_states).view(per_head)).transpose(1, 2)
        v = a.v_proj(hidden_states).view(per_head).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        key_cache, value_cache = cache.update(k, v, a.layer_idx)
        out = torch.ops.xinfer.batched_flash_attention(q, key_cache, value_cache, cache.offsets, cache.cuda_offsets,
                                                       cache.blocks, a.scaling)
        out = out.transpose(1, 2).reshape(*batch_shape, -1).contiguous()
        return a.o_proj(out * torch.sigmoid(gate)), None


def model_family(model):
    """'qwen3' or 'qwen35' from the model's configuration type."""
    model_type = model.config.model_type
    if model_type == "qwen3":
        return "qwen3"
    if model_type in ("qwen3_5_text", "qwen3_5"):
        return "qwen35"
    raise ValueError(f"Unsupported model type {model_type!r}; expected Qwen3 or Qwen3.5")


def install_attention(model, *, fused=False):
    """Replace each full-attention module of ``model`` by its adapter, keeping the original weights.

    Every replacement is built (and checked) before any layer changes, so a
    rejected model stays untouched; layers that already hold an adapter are
    left as they are.  ``fused`` selects the fused Qwen3 form.
    """
    family = model_family(model)
    require(not (fused and family == "qwen35"),
            "The fused norm/rope step covers Qwen3 (full-width rotary, plain RMSNorm weights)")
    replacements = []
    for index, layer in enumerate(model.model.layers):
        if family == "qwen35" and model.config.layer_types[index] != "full_attention":
            continue
        if isinstance(layer.self_attn, (Qwen3FlashAttention, Qwen35FlashAttention)):
            continue
        adapter = Qwen3FlashAttention(layer.self_attn, fused=fused) if family == "qwen3" else \
            Qwen35FlashAttention(layer.self_attn)
        adapter.train(layer.self_attn.training)
        replacements.append((layer, adapter))
    load_attention_ops(model=family)
    for layer, adapter in replacements:
        layer.self_attn = adapter
    return model


def rotary_tables(model, hidden, positions):
    """cos/sin [B, T, rotary_dim] of the step's positions, in the hidden dtype.

    Computed over the flattened positions, so that no batch dimension of one
    is specialised during export.  Qwen3 uses its rotary module as is.  For
    Qwen3.5 text, whose three multimodal position grids are equal, the
    interleaved multimodal rotary reduces to the plain one: angles = position
    * inv_freq, duplicated over the two halves, times attention_scaling.
    """
    rotary = model.model.rotary_emb
    if model_family(model) == "qwen3":
        tables = rotary(hidden, positions.reshape(1, -1))
        return tuple(t.reshape(*positions.shape, -1) for t in tables)
    angles = positions.reshape(-1, 1).float() * rotary.inv_freq.float()[None, :]
    angles = torch.cat((angles, angles), dim=-1)
    scale = rotary.attention_scaling
    return tuple((f(angles) * scale).to(hidden.dtype).reshape(*positions.shape, -1) for f in (torch.cos, torch.sin))


class ModelStep(torch.nn.Module):
    """One inference step of a causal LM whose attention layers run the native operators.

    forward(input_ids [B, T] int64, cache_position [B, T] int64, kv (2 tensors
    per layer, [B, Hkv, C, D] bf16, mutated in place), kv_lengths [B] and
    query_lengths [B] CPU int32) -> logits [B, vocab] of each row's last real
    token, zero for rows without new tokens.  The embedding, the unchanged
    decoder layers, the final norm and the LM head are the model's own; the
    loop passes no attention mask, since causality lives in the cache lengths.
    Rows are right-padded: tokens past a row's count are computed but never
    appended, and their outputs are not read.
    """

    def __init__(self, model, *, fused=False):
        super().__init__()
        family = model_family(model)
        if family == "qwen35":
            require(all(kind == "full_attention" for kind in model.config.layer_types),
                    "Linear-attention layers are not attention operators of this library")
        install_attention(model, fused=fused)
        self.model = model
        self.eval()

    def forward(self, input_ids, cache_position, kv, kv_lengths, query_lengths):
        cache = KVCache(kv, cache_position, kv_lengths, query_lengths)
        base = self.model.model
        hidden = base.embed_tokens(input_ids)
        rotary = rotary_tables(self.model, hidden, cache_position)
        for layer in base.layers:
            out = layer(hidden, attention_mask=None, position_ids=cache_position, past_key_values=cache,
                        cache_position=cache_position, position_embeddings=rotary, use_cache=True)
            hidden = out[0] if isinstance(out, tuple) else out
        hidden = base.norm(hidden)
        counts = query_lengths.to(device=hidden.device, dtype=torch.int64)
        last = hidden.gather(1, (counts - 1).clamp_min(0)[:, None, None].expand(-1, 1, hidden.shape[-1]))
        logits = self.model.lm_head(last)[:, 0, :]
        return logits.masked_fill(counts[:, None] == 0, 0)
