"""The adapters' contract on the CPU: installation and what they refuse.

Counterpart of compiler/qwen3/tests/test_attention.py:178-240 (unsupported
inputs raise ValueError; installation keeps the original modules and their
parameters, and a second installation changes nothing).  No operator runs:
every refusal happens before the first native call, so small transformers
models on the CPU suffice.
"""

import pytest
import torch

from xinfer_amd.adapters import (KVCache, ModelStep, Qwen35FlashAttention, Qwen3FlashAttention, install_attention,
                                 rotary_tables)


def qwen3_model(layers=2):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Config, Qwen3ForCausalLM

    config = Qwen3Config(vocab_size=32, hidden_size=64, intermediate_size=128, num_hidden_layers=layers,
                         num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=64,
                         use_sliding_window=False)
    config._attn_implementation = "sdpa"
    torch.manual_seed(0)
    return Qwen3ForCausalLM(config).eval().requires_grad_(False)


def qwen35_model(layer_types=("full_attention", "full_attention")):
    from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM, Qwen3_5TextConfig

    config = Qwen3_5TextConfig(vocab_size=32, hidden_size=64, intermediate_size=128, num_hidden_layers=len(layer_types),
                               num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                               layer_types=list(layer_types), max_position_embeddings=64)
    config._attn_implementation = "sdpa"
    torch.manual_seed(0)
    return Qwen3_5ForCausalLM(config).eval().requires_grad_(False)


@pytest.mark.parametrize("family", ["qwen3", "qwen35"])
def test_installation_keeps_modules_and_parameters(family):
    model = qwen3_model() if family == "qwen3" else qwen35_model()
    originals = [layer.self_attn for layer in model.model.layers]
    pointers = {name: p.data_ptr() for name, p in model.named_parameters()}
    install_attention(model)
    adapter = Qwen3FlashAttention if family == "qwen3" else Qwen35FlashAttention
    for layer, original in zip(model.model.layers, originals):
        assert isinstance(layer.self_attn, adapter) and layer.self_attn.original is original
    # The same parameters under the adapters' names: nothing copied.
    after = {name.replace("self_attn.original.", "self_attn."): p.data_ptr() for name, p in model.named_parameters()}
    assert after == pointers
    adapters = [layer.self_attn for layer in model.model.layers]
    install_attention(model)
    assert all(layer.self_attn is a for layer, a in zip(model.model.layers, adapters))


def test_hybrid_models_keep_their_linear_attention_and_refuse_a_step():
    model = qwen35_model(("linear_attention", "full_attention"))
    linear, full = model.model.layers[0].linear_attn, model.model.layers[1].self_attn
    with pytest.raises(ValueError, match="Linear-attention"):
        ModelStep(model)
    assert model.model.layers[1].self_attn is full
    install_attention(model)
    assert model.model.layers[0].linear_attn is linear
    assert isinstance(model.model.layers[1].self_attn, Qwen35FlashAttention)


def test_invalid_modules_and_forms_are_refused():
    with pytest.raises(ValueError, match="Qwen3Attention"):
        Qwen3FlashAttention(torch.nn.Linear(2, 2))
    with pytest.raises(ValueError, match="Qwen3.5"):
        Qwen35FlashAttention(qwen3_model().model.layers[0].self_attn)
    model = qwen35_model()
    before = [layer.self_attn for layer in model.model.layers]
    with pytest.raises(ValueError, match="fused"):
        install_attention(model, fused=True)
    assert [layer.self_attn for layer in model.model.layers] == before
    bad = qwen3_model()
    bad.model.layers[1].self_attn.k_norm.variance_epsilon = 1e-5
    with pytest.raises(ValueError, match="epsilon"):
        install_attention(bad, fused=True)
    assert not any(isinstance(layer.self_attn, Qwen3FlashAttention) for layer in bad.model.layers)
    with pytest.raises(ValueError, match="Unsupported model type"):
        install_attention(_fake_model())


def _fake_model():
    model = torch.nn.Module()
    model.config = type("Config", (), {"model_type": "llama"})()
    return model


@pytest.mark.parametrize("family", ["qwen3", "qwen35"])
def test_unsupported_inputs_are_rejected(family):
    model = qwen3_model() if family == "qwen3" else qwen35_model()
    install_attention(model)
    adapter = model.model.layers[0].self_attn
    config = model.config
    hidden = torch.zeros(1, 1, config.hidden_size, dtype=torch.float32)
    positions = torch.zeros(1, 1, dtype=torch.int64)
    kv = tuple(torch.zeros(1, config.num_key_value_heads, 8, config.head_dim) for _ in range(2 * len(model.model.layers)))
    cache = KVCache(kv, positions, torch.tensor([1], dtype=torch.int32), torch.tensor([1], dtype=torch.int32))
    arguments = dict(position_embeddings=rotary_tables(model, hidden, positions), past_key_values=cache,
                     cache_position=positions)
    cases = (
        ("mask", {"attention_mask": torch.zeros(1, 1, 1, 8)}, "attention masks"),
        ("cache", {"past_key_values": object()}, "KVCache"),
        ("no cache", {"past_key_values": None}, "KVCache"),
        ("positions", {"cache_position": positions.clone()}, "position tensor"),
        ("attention weights", {"output_attentions": True}, "attention weights"),
        ("training", {}, "attention weights"),
    )
    try:
        for name, changes, message in cases:
            adapter.train(name == "training")
            with pytest.raises(ValueError, match=message):
                adapter(hidden, **(arguments | changes))
    finally:
        adapter.eval()


def test_qwen35_rotary_tables_equal_the_multimodal_rotary():
    """With three equal position grids the interleaved multimodal rotary is the plain one."""
    model = qwen35_model()
    hidden = torch.zeros(2, 5, model.config.hidden_size)
    positions = torch.tensor([[0, 1, 2, 3, 4], [7, 8, 9, 10, 11]])
    cos, sin = rotary_tables(model, hidden, positions)
    ref_cos, ref_sin = model.model.rotary_emb(hidden, positions)
    assert cos.shape == ref_cos.shape == (2, 5, model.config.head_dim // 4)
    torch.testing.assert_close(cos, ref_cos, rtol=0, atol=1e-6)
    torch.testing.assert_close(sin, ref_sin, rtol=0, atol=1e-6)
