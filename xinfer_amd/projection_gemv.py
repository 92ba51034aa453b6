"""Singleton decoder projections as one native launch.

Python entry of ``xinfer::projection_gemv`` (libxinfer_attention_ops.so, HIP
kernel xinfer_amd/csrc/gemv.hip), with the reference's name, arguments,
checks and messages (compiler/common/kernels/projection_gemv.py:35-62), where
it is a Triton op.  The graph pass that selects it
(compiler/common/passes/projection_gemv.py) is unchanged: it retargets
``aten.linear`` nodes to ``torch.ops.xinfer.projection_gemv``.
"""

from xinfer_amd.attention import load_attention_ops


def projection_gemv(x, weight):
    """One input row times the weight's transpose, shaped as F.linear shapes it; inputs stay unchanged.

    ``x``: [1, ..., 1, k] with unit last stride; ``weight``: contiguous [n, k];
    both bf16 or both fp32, on one GPU.  Accumulates in fp32.  Invalid inputs
    raise ValueError with the reference's messages.
    """
    import torch

    if not hasattr(torch.ops.xinfer, "projection_gemv"):
        load_attention_ops(model="qwen35")
    return torch.ops.xinfer.projection_gemv(x, weight)
