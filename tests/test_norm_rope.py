"""The fused step before the attention operator: oracle pinning (CPU) and the
HIP kernel's parity (GPU).

The reference runs this step as eager modules (compiler/qwen3/adapters/attention.py:44-51):
transformers' Qwen3RMSNorm for q_norm / k_norm, apply_rotary_pos_emb, then
KVCache.update, i.e. append_kv_batched (compiler/qwen3/model.py:49-52).  The
CPU tests pin oracle/norm_rope.py against those same transformers functions
on CPU tensors, against closed forms, and against planted mistakes.  The GPU
tests compare the native operator with the eager modules on the GPU and with
the oracle: the rotated query and key to two bf16 units in the last place in
under 1% of the elements (the norm's fp32 sum of squares may round differently
in its last bit, which can flip the rounding of a normalised element, and the
rotation mixes two of them into each output), the value
and every untouched cache slot bit for bit, and the attention output computed
from the fused step's results against the one from the eager step.
"""

import numpy as np
import pytest
import torch

from oracle import norm_rope as ref


def bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def ulp_distance(a, b):
    """|a - b| in bf16 units in the last place (finite values of one sign order)."""
    def key(x):
        x = np.asarray(x, dtype=np.uint16).astype(np.int32)
        return np.where(x & 0x8000, 0x8000 - (x & 0x7FFF), 0x8000 + x)
    return np.abs(key(a) - key(b))


def hf_modules(dim, eps, weight):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm

    norm = Qwen3RMSNorm(dim, eps=eps).to(torch.bfloat16)
    with torch.no_grad():
        norm.weight.copy_(weight)
    return norm


def draw(seed, batch, tokens, heads, kv_heads, dim):
    g = torch.Generator().manual_seed(seed)
    q = (torch.randn(batch, tokens, heads, dim, generator=g) * 3).to(torch.bfloat16)
    k = (torch.randn(batch, tokens, kv_heads, dim, generator=g) * 3).to(torch.bfloat16)
    v = torch.randn(batch, tokens, kv_heads, dim, generator=g).to(torch.bfloat16)
    qw = (1 + 0.2 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(dim, generator=g)).to(torch.bfloat16)
    angle = torch.rand(batch, tokens, dim // 2, generator=g, dtype=torch.float64) * 100
    angle = torch.cat([angle, angle], dim=-1)
    cos, sin = angle.cos().to(torch.bfloat16), angle.sin().to(torch.bfloat16)
    return q, k, v, qw, kw, cos, sin


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_rope_stage_matches_transformers_bit_for_bit(dim):
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb

    q, k, _, _, _, cos, sin = draw(1, 2, 5, 4, 2, dim)
    qh, kh = q.transpose(1, 2), k.transpose(1, 2)
    eq, ek = apply_rotary_pos_emb(qh, kh, cos, sin)
    cs, sn = bits(cos)[:, None], bits(sin)[:, None]
    assert np.array_equal(ref.rope(bits(qh), cs, sn), bits(eq))
    assert np.array_equal(ref.rope(bits(kh), cs, sn), bits(ek))


@pytest.mark.parametrize("dim", [64, 128, 256])
def test_norm_stage_matches_transformers_within_one_ulp(dim):
    q, _, _, qw, _, _, _ = draw(2, 3, 17, 8, 4, dim)
    norm = hf_modules(dim, 1e-6, qw)
    with torch.no_grad():
        expected = bits(norm(q))
    actual = ref.rms_norm(bits(q), bits(qw), 1e-6)
    distance = ulp_distance(actual, expected)
    assert distance.max() <= 1
    assert (distance > 0).mean() < 0.01


def test_closed_forms():
    dim = 128
    # A constant row normalises to sign(c) / sqrt(1 + eps / c^2), i.e. +-1 here, then the weight.
    row = np.full((1, dim), ref.f32_to_bf16(np.float32(2.5)), dtype=np.uint16)
    w = ref.f32_to_bf16(np.linspace(0.5, 1.5, dim, dtype=np.float32))
    assert np.array_equal(ref.rms_norm(row, w, 0.0), w[None])
    # cos = 1, sin = 0 is the identity; cos = 0, sin = 1 is rotate_half.
    x = ref.f32_to_bf16(np.random.default_rng(0).standard_normal((3, dim)).astype(np.float32))
    one, zero = ref.f32_to_bf16(np.ones(dim, np.float32)), ref.f32_to_bf16(np.zeros(dim, np.float32))
    assert np.array_equal(ref.rope(x, one, zero), x)
    xf = ref.bf16_to_f32(x)
    rotated = np.concatenate([-xf[:, dim // 2:], xf[:, : dim // 2]], axis=1)
    assert np.array_equal(ref.rope(x, zero, one), ref.f32_to_bf16(rotated))


def test_planted_mistakes_fail():
    """Variants with a plausible mistake must disagree with transformers."""
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb

    dim = 128
    q, k, _, qw, _, cos, sin = draw(3, 1, 9, 4, 2, dim)
    qh = q.transpose(1, 2)
    eq, _ = apply_rotary_pos_emb(qh, k.transpose(1, 2), cos, sin)
    cs, sn = ref.bf16_to_f32(bits(cos)[:, None]), ref.bf16_to_f32(bits(sin)[:, None])
    x = ref.bf16_to_f32(bits(qh))
    half = dim // 2

    def finish(rot):
        return ref.f32_to_bf16(ref.round_bf16(x * cs) + ref.round_bf16(rot * sn))

    wrong_sign = finish(np.concatenate([x[..., half:], -x[..., :half]], axis=-1))
    wrong_pairing = finish(np.concatenate([-x[..., 1::2], x[..., 0::2]], axis=-1))
    assert not np.array_equal(wrong_sign, bits(eq))
    assert not np.array_equal(wrong_pairing, bits(eq))
    norm = hf_modules(dim, 1e-6, qw)
    with torch.no_grad():
        expected = bits(norm(q))
    no_weight = ref.rms_norm(bits(q), ref.f32_to_bf16(np.ones(dim, np.float32)), 1e-6)
    assert ulp_distance(no_weight, expected).max() > 1
    tiny = (torch.randn(1, 2, 2, dim) * 1e-4).to(torch.bfloat16)
    with torch.no_grad():
        expected_tiny = bits(norm(tiny))
    assert ulp_distance(ref.rms_norm(bits(tiny), bits(qw), 0.0), expected_tiny).max() > 1


def test_append_matches_a_brute_force_loop():
    batch, tokens, heads, kv_heads, dim, capacity = 3, 4, 4, 2, 64, 16
    q, k, v, qw, kw, cos, sin = draw(4, batch, tokens, heads, kv_heads, dim)
    positions = np.array([[3, 4, 5, 6], [0, 1, 99, 99], [15, 16, -1, 2]])
    cu_query = np.array([0, 4, 6, 10])
    ck = np.zeros((batch, kv_heads, capacity, dim), np.uint16)
    cv = np.zeros_like(ck)
    q_out = ref.norm_rope_append(bits(q), bits(k), bits(v), bits(qw), bits(kw), 1e-6, bits(cos), bits(sin),
                                 positions, cu_query, ck, cv)
    k_rot = ref.rope(ref.rms_norm(bits(k), bits(kw), 1e-6), bits(cos)[:, :, None], bits(sin)[:, :, None])
    ek, ev = np.zeros_like(ck), np.zeros_like(cv)
    for r, valid in enumerate([(0, 1, 2, 3), (0, 1), (0, 3)]):  # row 2: position 16 and -1 are skipped
        for t in valid:
            for h in range(kv_heads):
                ek[r, h, positions[r, t]] = k_rot[r, t, h]
                ev[r, h, positions[r, t]] = bits(v)[r, t, h]
    assert np.array_equal(ck, ek) and np.array_equal(cv, ev)
    assert q_out.shape == (batch, heads, tokens, dim)


# ----------------------------------------------------------------------------- GPU


def eager_step(q, k, v, qw, kw, eps, cos, sin, positions, cu_query, cache_key, cache_value):
    """The reference adapter's step (attention.py:44-51) with transformers' modules."""
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
    from xinfer_amd.kv_cache import append_kv_batched

    dim = q.shape[-1]
    q_norm, k_norm = hf_modules(dim, eps, qw.cpu()).to(q.device), hf_modules(dim, eps, kw.cpu()).to(q.device)
    qh = q_norm(q).transpose(1, 2)
    kh = k_norm(k).transpose(1, 2)
    vh = v.transpose(1, 2)
    qh, kh = apply_rotary_pos_emb(qh, kh, cos, sin)
    append_kv_batched(kh, vh, positions, cu_query, cache_key, cache_value)
    return qh


@pytest.mark.gpu
@torch.inference_mode()
@pytest.mark.parametrize("batch,tokens,heads,kv_heads,dim", [
    (1, 512, 16, 8, 128),   # cfg2 chunk
    (8, 1, 16, 8, 128),     # cfg3 decode step
    (3, 37, 16, 4, 256),    # Qwen3.5-style head dim
    (2, 5, 8, 8, 64),
])
def test_fused_step_matches_the_eager_modules(gpu_ops, batch, tokens, heads, kv_heads, dim):
    from attn_helpers import assert_close_rows, log, reference_attention
    from xinfer_amd.attention import batched_attention_metadata
    from xinfer_amd.norm_rope import qk_norm_rope_append

    log(f"norm/rope/append batch={batch} tokens={tokens} heads={heads}/{kv_heads} dim={dim}")
    capacity = 4096
    q, k, v, qw, kw, cos, sin = (t.cuda() for t in draw(7, batch, tokens, heads, kv_heads, dim))
    counts = [tokens if r % 2 == 0 else max(tokens // 2, 0) for r in range(batch)]
    starts = [100 + 17 * r for r in range(batch)]
    lengths = [s + c for s, c in zip(starts, counts)]
    positions = torch.stack([torch.arange(s, s + tokens) for s in starts]).cuda()
    for r, count in enumerate(counts):
        positions[r, count:] = capacity + 100  # padded positions are never dereferenced
    host, cu, blocks = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), q.device)
    base_k = torch.randn(batch, kv_heads, capacity, dim, device="cuda").to(torch.bfloat16)
    base_v = torch.randn_like(base_k)
    fused_k, fused_v, eager_k, eager_v = base_k.clone(), base_v.clone(), base_k.clone(), base_v.clone()
    inputs = [t.clone() for t in (q, k, v, qw, kw, cos, sin, positions)]

    q_fused = qk_norm_rope_append(q, k, v, qw, kw, 1e-6, cos, sin, positions, cu[0], fused_k, fused_v)
    q_eager = eager_step(q, k, v, qw, kw, 1e-6, cos, sin, positions, cu[0], eager_k, eager_v)
    assert all(torch.equal(a, b) for a, b in zip(inputs, (q, k, v, qw, kw, cos, sin, positions)))
    assert q_fused.is_contiguous() and q_fused.shape == (batch, heads, tokens, dim)

    def check_close(actual, expected, what):
        distance = ulp_distance(actual, expected)
        worst, share = int(distance.max()), float((distance > 0).mean())
        log(f"  {what}: {int((distance > 0).sum())} of {distance.size} elements differ, at most {worst} ulp")
        assert worst <= 2 and share < 0.01, (what, worst, share)

    check_close(bits(q_fused.cpu()), bits(q_eager.cpu()), "query vs eager")
    check_close(bits(fused_k.cpu()), bits(eager_k.cpu()), "key cache vs eager")
    assert torch.equal(fused_v, eager_v)
    written = torch.zeros(batch, capacity, dtype=torch.bool)
    for r, (s, c) in enumerate(zip(starts, counts)):
        written[r, s:s + c] = True
    untouched = ~written[:, None, :].expand(-1, kv_heads, -1)
    assert torch.equal(fused_k.cpu()[untouched], base_k.cpu()[untouched])
    assert torch.equal(fused_v.cpu()[untouched], base_v.cpu()[untouched])

    # Against the oracle on the CPU.
    ck, cv = bits(base_k.cpu()).copy(), bits(base_v.cpu()).copy()
    q_ref = ref.norm_rope_append(bits(q.cpu()), bits(k.cpu()), bits(v.cpu()), bits(qw.cpu()), bits(kw.cpu()), 1e-6,
                                 bits(cos.cpu()), bits(sin.cpu()), positions.cpu().numpy(), cu[0].cpu().numpy(),
                                 ck, cv)
    check_close(bits(q_fused.cpu()), q_ref, "query vs oracle")
    check_close(bits(fused_k.cpu()), ck, "key cache vs oracle")
    assert np.array_equal(bits(fused_v.cpu()), cv)

    # The attention output from the fused step against the one from the eager step.
    op = gpu_ops.batched_flash_attention.default
    scale = dim**-0.5
    actual = op(q_fused, fused_k, fused_v, host, cu, blocks, scale)
    expected = reference_attention(q_eager, eager_k, eager_v, counts, lengths, scale)
    assert_close_rows(actual, expected, counts)


@pytest.mark.gpu
@torch.inference_mode()
def test_fused_step_accepts_strided_projections_and_rejects_bad_inputs(gpu_ops):
    from xinfer_amd.norm_rope import qk_norm_rope_append

    batch, tokens, heads, kv_heads, dim = 2, 6, 16, 8, 128
    q, k, v, qw, kw, cos, sin = (t.cuda() for t in draw(9, batch, tokens, heads, kv_heads, dim))
    # One fused QKV projection, split by views (non-contiguous heads).
    qkv = torch.cat([q.flatten(2), k.flatten(2), v.flatten(2)], dim=-1)
    qs = qkv[..., : heads * dim].view(batch, tokens, heads, dim)
    ks = qkv[..., heads * dim:(heads + kv_heads) * dim].view(batch, tokens, kv_heads, dim)
    vs = qkv[..., (heads + kv_heads) * dim:].view(batch, tokens, kv_heads, dim)
    positions = torch.arange(tokens).repeat(batch, 1).cuda()
    cu = torch.tensor([0, tokens, 2 * tokens], dtype=torch.int32, device="cuda")
    caches = [torch.zeros(batch, kv_heads, 64, dim, device="cuda", dtype=torch.bfloat16) for _ in range(4)]
    a = qk_norm_rope_append(qs, ks, vs, qw, kw, 1e-6, cos, sin, positions, cu, caches[0], caches[1])
    b = qk_norm_rope_append(q, k, v, qw, kw, 1e-6, cos, sin, positions, cu, caches[2], caches[3])
    assert torch.equal(a, b) and torch.equal(caches[0], caches[2]) and torch.equal(caches[1], caches[3])
    with pytest.raises(RuntimeError, match="RMSNorm epsilon"):
        qk_norm_rope_append(q, k, v, qw, kw, -1.0, cos, sin, positions, cu, caches[0], caches[1])
    with pytest.raises(RuntimeError, match="Expected q"):
        qk_norm_rope_append(q, k, v, qw, kw, 1e-6, cos[..., :64], sin[..., :64], positions, cu, caches[0], caches[1])
    with pytest.raises(RuntimeError, match="contiguous KV caches"):
        qk_norm_rope_append(q, k, v, qw, kw, 1e-6, cos, sin, positions, cu, caches[0].transpose(2, 3), caches[1])
