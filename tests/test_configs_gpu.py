"""Parity of one hot-path step (KV append + attention) on the five measured configurations.

Inputs are the seeded CPU draws of xinfer_amd.workloads (identical bits for the
GPU and the CPU oracle).  Gates:

* the KV caches after the append equal, bit for bit, the caches the workload
  builds on the CPU by slice assignment of the new tokens (every untouched
  slot included);
* attention outputs are within max-abs 2e-2 and mean-abs 2e-3 of the float64
  oracle;
* the error is no worse than the reference path's own bf16 error: torch SDPA
  on bf16 tensors with the explicit lower-right mask (the adapted eager
  attention) on the device's flash-family kernels, measured on the same rows
  and inputs.  On every input the bench times, both the worst and the mean
  absolute error must be at or below the reference path's.

More draws of the two prefill configurations (cfg2 seeds 0-5, cfg5 seeds
0-3) are held to the same bar across draws: per draw the mean absolute error
at or below the reference path's and the absolute gates; per configuration
the worst error over its draws at or below the reference path's worst over
the same draws.  Per draw, the worst error of both paths is an output
element about half a bf16 step from its exact value, whose side of a
rounding midpoint the weights' bf16 rounding decides in either path, so it
is compared over the draws rather than draw by draw; each draw's ratio is
logged.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel
from torch.nn.attention.bias import causal_lower_right

from attn_helpers import MAX_ABS, MEAN_ABS, log
from oracle import attention as oracle
from xinfer_amd import workloads
from xinfer_amd.attention import batched_attention_metadata, cache_extent

pytestmark = pytest.mark.gpu

# Our error may exceed the bf16 reference path's error by at most this factor:
# BASELINE.json asks for "no worse than the reference's own bf16 error".
BF16_SLACK = 1.0


def row_slices(inputs, r, length, count):
    k = inputs["k_after"][r : r + 1, :, :length]
    v = inputs["v_after"][r : r + 1, :, :length]
    q = inputs["q"][r : r + 1, :, :count]
    return q, k, v


def bf16_reference(q, k, v, count, length, scale):
    """The reference path's own bf16 result on the same inputs.

    torch SDPA on bf16 device tensors with the explicit lower-right causal mask,
    restricted to the flash / memory-efficient kernels (ATen's FlashAttention
    family, which the reference operator calls; the MATH path is never used on
    the device).  Falls back to CPU SDPA MATH on bf16 (which keeps P in fp32, a
    stricter bar) if no device kernel accepts the shapes.  Returns (output, source).
    """
    group = q.shape[1] // k.shape[1]
    try:
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            out = F.scaled_dot_product_attention(
                q.cuda(), k.repeat_interleave(group, 1).cuda(), v.repeat_interleave(group, 1).cuda(),
                attn_mask=causal_lower_right(count, length), scale=scale)
        torch.cuda.synchronize()
        return out.cpu(), "device flash/efficient SDPA"
    except RuntimeError:
        mask = torch.arange(length)[None, :] <= torch.arange(length - count, length)[:, None]
        with sdpa_kernel(SDPBackend.MATH):
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True, scale=scale)
        return out, "CPU SDPA MATH"


def run_step(gpu_ops, w, inputs):
    device = "cuda"
    q = inputs["q"].to(device)
    k = inputs["k"].to(device)
    v = inputs["v"].to(device)
    counts = torch.tensor(w.counts, dtype=torch.int32)
    lengths = torch.tensor(w.lengths, dtype=torch.int32)
    host, cu, blocks = batched_attention_metadata(lengths, counts, device)
    if w.append:
        new_k = inputs["new_k"].to(device)
        new_v = inputs["new_v"].to(device)
        positions = inputs["positions"].to(device)
        gpu_ops.append_kv_batched(new_k, new_v, positions, cu[0], k, v)
    if w.op == "flash":
        out = gpu_ops.flash_attention(q, k, v, cache_extent(w.lengths[0]), w.scale)
    else:
        out = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, w.scale)
    torch.cuda.synchronize()
    return out.cpu(), k, v


# Every input the bench times (cfg3 seeds 0-7 among them) and a second draw
# of each prefill configuration, each under the same strict gate.
CASES = [(1, 0), (2, 0), (2, 1), (3, 0), (3, 1), (3, 2), (3, 3), (3, 4), (3, 5), (3, 6), (3, 7), (4, 0),
         (5, 0), (5, 1)]


def draw_errors(gpu_ops, index, seed):
    """(ours, reference path) error statistics of one draw against the float64 oracle,
    after checking the appended caches bit for bit."""
    w = workloads.config(index, seed)
    log(f"config {w.name} seed {seed}: B={w.batch} Hq={w.heads} Hkv={w.kv_heads} D={w.dim} C={w.capacity} "
        f"counts={w.counts} lengths={w.lengths}")
    inputs = workloads.make_inputs(w)
    out, k_gpu, v_gpu = run_step(gpu_ops, w, inputs)
    if w.append:
        # Bit-exact cache after the append, including every untouched slot.
        assert torch.equal(k_gpu.cpu().view(torch.int16), inputs["k_after"].view(torch.int16))
        assert torch.equal(v_gpu.cpu().view(torch.int16), inputs["v_after"].view(torch.int16))
    del k_gpu, v_gpu
    # Every row is compared three ways on the same elements: ours and the bf16
    # reference path, each against the float64 oracle.
    worst = dict(max_abs=0.0, sum_abs=0.0, n=0, ref_max_abs=0.0, ref_sum_abs=0.0)
    for r, (count, length) in enumerate(zip(w.counts, w.lengths)):
        assert torch.count_nonzero(out[r, :, count:]).item() == 0
        q, k, v = row_slices(inputs, r, length, count)
        expected = oracle.attention(*(oracle.bf16_to_f32(x.view(torch.int16).numpy().view(np.uint16)).astype(np.float64)
                                      for x in (q, k, v)), [count], [length], w.scale)
        delta = np.abs(out[r : r + 1, :, :count].float().numpy().astype(np.float64) - expected)
        worst["max_abs"] = max(worst["max_abs"], float(delta.max()))
        worst["sum_abs"] += float(delta.sum())
        worst["n"] += delta.size
        ref, source = bf16_reference(q, k, v, count, length, w.scale)
        ref_delta = np.abs(ref.float().numpy().astype(np.float64) - expected)
        worst["source"] = source
        worst["ref_max_abs"] = max(worst["ref_max_abs"], float(ref_delta.max()))
        worst["ref_sum_abs"] += float(ref_delta.sum())
    stats = dict(max_abs=worst["max_abs"], mean_abs=worst["sum_abs"] / worst["n"], ref_max_abs=worst["ref_max_abs"],
                 ref_mean_abs=worst["ref_sum_abs"] / worst["n"], source=worst["source"])
    log(f"  errors vs float64 oracle: max_abs={stats['max_abs']:.3e} mean_abs={stats['mean_abs']:.3e}; "
        f"bf16 reference path ({stats['source']}): max_abs={stats['ref_max_abs']:.3e} "
        f"mean_abs={stats['ref_mean_abs']:.3e}; ratios max {stats['max_abs'] / stats['ref_max_abs']:.3f} "
        f"mean {stats['mean_abs'] / stats['ref_mean_abs']:.3f}")
    assert stats["max_abs"] <= MAX_ABS
    assert stats["mean_abs"] <= MEAN_ABS
    return stats


@pytest.mark.parametrize("index,seed", CASES, ids=[f"cfg{i}_seed{s}" for i, s in CASES])
@torch.inference_mode()
def test_config_parity(gpu_ops, index, seed):
    stats = draw_errors(gpu_ops, index, seed)
    assert stats["mean_abs"] <= BF16_SLACK * stats["ref_mean_abs"]
    assert stats["max_abs"] <= BF16_SLACK * stats["ref_max_abs"]


# Prefill configurations and the draws held to the bar across draws.
DRAWS = {2: range(6), 5: range(4)}


@pytest.mark.parametrize("index", sorted(DRAWS), ids=[f"cfg{i}" for i in sorted(DRAWS)])
@torch.inference_mode()
def test_prefill_draws_against_the_reference_error(gpu_ops, index):
    draws = [draw_errors(gpu_ops, index, seed) for seed in DRAWS[index]]
    for seed, stats in zip(DRAWS[index], draws):
        assert stats["mean_abs"] <= BF16_SLACK * stats["ref_mean_abs"], (index, seed, stats)
    ours, reference = max(d["max_abs"] for d in draws), max(d["ref_max_abs"] for d in draws)
    log(f"cfg{index} seeds {list(DRAWS[index])}: worst max_abs {ours:.3e} against the reference path's "
        f"{reference:.3e} (ratio {ours / reference:.3f}); per-draw max ratios "
        f"{[round(d['max_abs'] / d['ref_max_abs'], 3) for d in draws]}")
    assert ours <= BF16_SLACK * reference


@torch.inference_mode()
def test_step_is_deterministic(gpu_ops):
    """Same inputs, same bits: the schedule depends only on lengths (cfg3, seed 0)."""
    w = workloads.config(3, 0)
    inputs = workloads.make_inputs(w)
    log(f"determinism {w.name}")
    first, _, _ = run_step(gpu_ops, w, inputs)
    second, _, _ = run_step(gpu_ops, w, inputs)
    assert torch.equal(first.view(torch.int16), second.view(torch.int16))
