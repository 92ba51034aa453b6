"""Synthetic workloads of the attention hot path: the five measured configurations.

Shapes follow Qwen3-0.6B (16 query / 8 KV heads, head dim 128) and the
Qwen3.5-4B full-attention layer (16 / 4, head dim 256).  Inputs are drawn on
the CPU from ``torch.Generator().manual_seed(seed)`` in a fixed order --
lengths, then Q, then K over the full capacity, then V, then the new chunk's
K and V -- as N(0, 1) fp32 cast to bf16, so every consumer (GPU kernels, the
CPU oracle, the CPU SDPA baseline) sees identical bits.

A step of the hot path is one KV append of each row's new tokens followed by
one attention call over the populated prefixes (the adapters' order,
compiler/qwen3/adapters/attention.py:49-60).
"""

from __future__ import annotations

from dataclasses import dataclass, field
import math

LOG16, LOG16384 = math.log(16), math.log(16384)


@dataclass
class Workload:
    name: str
    kind: str                # "decode" (HBM-bound) or "prefill" (MFMA-bound)
    op: str                  # "flash" (uniform length) or "batched"
    heads: int
    kv_heads: int
    dim: int
    capacity: int
    counts: list             # new (real) query tokens per row
    prefixes: list           # populated keys before the new tokens, per row
    append: bool = True      # the step writes the new K/V into the cache first
    seed: int = 0
    description: str = ""
    lengths: list = field(init=False)

    def __post_init__(self):
        self.lengths = [p + n for p, n in zip(self.prefixes, self.counts)]

    @property
    def batch(self):
        return len(self.counts)

    @property
    def tokens(self):
        return max(self.counts)

    @property
    def scale(self):
        return self.dim ** -0.5

    def kv_bytes(self):
        """Decode algorithmic HBM bytes: sum_r 2 * L_r * Hkv * D * 2 (K and V, bf16)."""
        return sum(2 * length * self.kv_heads * self.dim * 2 for length in self.lengths)

    def flops(self):
        """Causal-exact attention FLOPs: 4 * Hq * D * sum_r (n_r p_r + n_r (n_r + 1) / 2)."""
        return 4 * self.heads * self.dim * sum(
            n * p + n * (n + 1) // 2 for n, p in zip(self.counts, self.prefixes)
        )

    def append_bytes(self):
        """KV append traffic: 2 * sum_r n_r * Hkv * D * 2 read + the same written."""
        if not self.append:
            return 0
        return 2 * (2 * sum(self.counts) * self.kv_heads * self.dim * 2)

    def summary(self):
        return {
            "workload": self.name,
            "batch": self.batch,
            "heads": self.heads,
            "kv_heads": self.kv_heads,
            "head_dim": self.dim,
            "capacity": self.capacity,
            "new_tokens": list(self.counts),
            "kv_lengths": list(self.lengths),
            "seed": self.seed,
        }


def ragged_decode_lengths(seed, batch=8):
    """L_r = floor(exp(U(ln 16, ln 16384))), U from torch.rand(float64)."""
    import torch

    generator = torch.Generator().manual_seed(seed)
    u = torch.rand(batch, dtype=torch.float64, generator=generator)
    return [int(x) for x in torch.floor(torch.exp(LOG16 + u * (LOG16384 - LOG16))).tolist()], generator


def ragged_prefill_lengths(seed, batch=8, capacity=16384):
    """n_r = randint(2, 513), p_r = min(randint(0, 15873), capacity - n_r)."""
    import torch

    generator = torch.Generator().manual_seed(seed)
    counts = torch.randint(2, 513, (batch,), generator=generator).tolist()
    prefixes = torch.randint(0, 15873, (batch,), generator=generator).tolist()
    prefixes = [min(p, capacity - n) for p, n in zip(prefixes, counts)]
    return counts, prefixes, generator


def config(index, seed=0):
    """Configuration ``index`` (1-based, as listed in BASELINE.json ``configs``)."""
    if index == 1:
        return Workload("cfg1_decode_b1_l1024", "decode", "flash", 16, 8, 128, 4096, [1], [1023],
                        append=False, seed=seed,
                        description="Qwen3-0.6B decode, B=1, L=1024, C=4096")
    if index == 2:
        return Workload("cfg2_prefill_b1_n512_p1536", "prefill", "batched", 16, 8, 128, 4096, [512],
                        [1536], seed=seed,
                        description="Qwen3-0.6B chunked prefill, 512 tokens at offset 1536, C=4096")
    if index == 3:
        lengths, _ = ragged_decode_lengths(seed)
        return Workload(f"cfg3_ragged_decode_b8_seed{seed}", "decode", "batched", 16, 8, 128, 16384,
                        [1] * 8, [length - 1 for length in lengths], seed=seed,
                        description="Qwen3-0.6B ragged decode, B=8, log-uniform L in [16,16384]")
    if index == 4:
        return Workload("cfg4_decode_b4_d256", "decode", "batched", 16, 4, 256, 16384, [1] * 4,
                        [1023, 4095, 8191, 16383], seed=seed,
                        description="Qwen3.5-4B decode, B=4, L={1K,4K,8K,16K}, C=16384")
    if index == 5:
        counts, prefixes, _ = ragged_prefill_lengths(seed)
        return Workload(f"cfg5_ragged_prefill_b8_seed{seed}", "prefill", "batched", 16, 4, 256, 16384,
                        counts, prefixes, seed=seed,
                        description="Qwen3.5-4B ragged prefill, B=8, n in [2,512], C=16384")
    raise ValueError(f"unknown config {index}")


def make_inputs(w: Workload):
    """Seeded CPU bf16 tensors of a workload.

    Returns dict(q [B,Hq,T,D], k/v caches [B,Hkv,C,D], new_k/new_v [B,Hkv,T,D],
    positions int64 [B,T] (padded tokens point past the capacity and are never
    read), counts, lengths).  ``k_after``/``v_after`` are the caches the attention
    reads: with the new tokens written in when the step appends, else the caches.
    """
    import torch

    generator = torch.Generator().manual_seed(w.seed)
    # Lengths are drawn first (their draw is consumed here to keep the order).
    if w.name.startswith("cfg3"):
        torch.rand(w.batch, dtype=torch.float64, generator=generator)
    elif w.name.startswith("cfg5"):
        torch.randint(2, 513, (w.batch,), generator=generator)
        torch.randint(0, 15873, (w.batch,), generator=generator)
    b, hq, hkv, t, d, c = w.batch, w.heads, w.kv_heads, w.tokens, w.dim, w.capacity

    def draw(*shape):
        return torch.randn(*shape, generator=generator, dtype=torch.float32).to(torch.bfloat16)

    q = draw(b, hq, t, d)
    k = draw(b, hkv, c, d)
    v = draw(b, hkv, c, d)
    new_k = draw(b, hkv, t, d)
    new_v = draw(b, hkv, t, d)
    positions = torch.full((b, t), c + 100, dtype=torch.int64)
    for r, (n, p) in enumerate(zip(w.counts, w.prefixes)):
        positions[r, :n] = torch.arange(p, p + n)
    k_after, v_after = k.clone(), v.clone()
    if w.append:
        for r, (n, p) in enumerate(zip(w.counts, w.prefixes)):
            k_after[r, :, p:p + n] = new_k[r, :, :n]
            v_after[r, :, p:p + n] = new_v[r, :, :n]
    return dict(q=q, k=k, v=v, new_k=new_k, new_v=new_v, positions=positions,
                k_after=k_after, v_after=v_after,
                counts=list(w.counts), lengths=list(w.lengths))
