"""Helpers shared by the GPU parity tests."""

import sys

import numpy as np
import torch

# BASELINE.json tolerance against an fp32 (here: float64 oracle or fp32 torch) reference.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def log(message):
    """Name the case before a GPU step, flushed, so a dying box still says where it was."""
    print(message, file=sys.stderr, flush=True)


def row_errors(actual, expected):
    """Row-wise errors as in compiler/common/tests/tensors.py:8-21, plus max/mean abs."""
    assert actual.shape == expected.shape, "Tensor shapes differ"
    assert torch.isfinite(actual).all() and torch.isfinite(expected).all(), "Nonfinite validation tensors"
    delta = actual - expected
    return dict(
        max_abs=delta.abs().max().item(),
        mean_abs=delta.abs().mean().item(),
        relative_l2=(delta.norm(dim=-1) / expected.norm(dim=-1).clamp_min(1e-12)).max().item(),
        peak_relative=(delta.abs().amax(dim=-1) / expected.abs().amax(dim=-1).clamp_min(1e-12)).max().item(),
    )


def reference_attention(q, k, v, counts, lengths, scale):
    """fp32 masked-softmax attention on the device (lower-right causal, GQA hq // G).

    The same formula as oracle/attention.py, used where the reference's tests use
    fp32 SDPA MATH on the GPU; operands are made contiguous before every matmul.
    """
    torch.backends.cuda.matmul.allow_tf32 = False
    out = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
    group = q.shape[1] // k.shape[1]
    for r, (count, length) in enumerate(zip(counts, lengths)):
        if count == 0:
            continue
        qr = q[r, :, :count].float().contiguous()
        kr = k[r, :, :length].float().repeat_interleave(group, 0)
        vr = v[r, :, :length].float().repeat_interleave(group, 0).contiguous()
        scores = torch.matmul(qr, kr.transpose(1, 2).contiguous()) * scale
        hidden = torch.arange(length, device=q.device)[None, :] > (
            length - count + torch.arange(count, device=q.device)
        )[:, None]
        scores.masked_fill_(hidden, float("-inf"))
        out[r, :, :count] = torch.matmul(scores.softmax(-1), vr)
    return out


def assert_close_rows(actual, expected, counts, *, relative_l2=0.01, peak_relative=0.05):
    """Reference test bounds per row (test_attention.py:112-113) plus max-abs <= 2e-2 and mean-abs <= 2e-3."""
    for r, count in enumerate(counts):
        if not count:
            continue
        errors = row_errors(actual[r : r + 1, :, :count].float().flatten(1),
                            expected[r : r + 1, :, :count].float().flatten(1))
        assert errors["relative_l2"] < relative_l2, errors
        assert errors["peak_relative"] <= peak_relative, errors
        assert errors["max_abs"] <= MAX_ABS, errors
        assert errors["mean_abs"] <= MEAN_ABS, errors


def to_numpy_f64(tensor):
    return tensor.detach().float().cpu().numpy().astype(np.float64)
