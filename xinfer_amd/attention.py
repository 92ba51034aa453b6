"""Load the native xinfer attention operators and register their shape contracts.

Mirror of the reference loader compiler/common/attention.py:1-112: the same
public names, arguments, errors and fake (meta) functions, so the reference's
adapters, exporter and tests bind to this module unchanged.  The library is the
hipcc-built libxinfer_attention_ops.so of this package (xinfer_amd/build.py),
which registers these operators in the `xinfer` namespace:

* ``flash_attention`` and ``batched_flash_attention`` -- read-only attention
  over each request's populated KV prefix (HIP kernels for gfx950);
* ``append_kv_batched`` -- the in-place KV-cache append, native instead of the
  reference's Triton op (compiler/common/kernels/kv_cache.py:45-72);
* ``batched_flash_attention_bthd`` -- ``batched_flash_attention`` with its
  output in [B,T,Hq,D] order (the adapter's reshape then needs no copy);
* ``batched_flash_attention_graph`` -- ``batched_flash_attention`` for steps
  that are captured once in a HIP graph and replayed while the lengths
  change: the kernels read the lengths from ``cuda_offsets`` (prefill shapes
  are planned by a kernel from them);
* ``projection_gemv`` -- the decoder's singleton projections, native instead
  of the reference's Triton op (compiler/common/kernels/projection_gemv.py);
* ``qk_norm_rope_append`` -- the step before the attention operator in one
  launch: q/k RMSNorm, rotary embedding and the KV append
  (compiler/qwen3/adapters/attention.py:44-51), see xinfer_amd/norm_rope.py.
"""

import os
from pathlib import Path

ROOT = Path(__file__).resolve().parent
ATTENTION_LIBRARY = "libxinfer_attention_ops.so"
# AOTInductor C-shim declarations: attention.py:10-16 of the reference, plus the
# append shim that a native (non-Triton) append needs.
ATTENTION_C_SHIM = """AOTITorchError aoti_torch_cuda_flash_attention(
    AtenTensorHandle q, AtenTensorHandle k, AtenTensorHandle v,
    AtenTensorHandle extent, double scale, AtenTensorHandle* output)"""
BATCHED_ATTENTION_C_SHIM = """AOTITorchError aoti_torch_cuda_batched_flash_attention(
    AtenTensorHandle q, AtenTensorHandle k, AtenTensorHandle v,
    AtenTensorHandle offsets, AtenTensorHandle cuda_offsets, AtenTensorHandle blocks,
    double scale, AtenTensorHandle* output)"""
APPEND_KV_C_SHIM = """AOTITorchError aoti_torch_cuda_append_kv_batched(
    AtenTensorHandle key, AtenTensorHandle value, AtenTensorHandle positions,
    AtenTensorHandle cu_query, AtenTensorHandle cache_key, AtenTensorHandle cache_value,
    AtenTensorHandle* unused_output)"""
BATCHED_BTHD_C_SHIM = """AOTITorchError aoti_torch_cuda_batched_flash_attention_bthd(
    AtenTensorHandle q, AtenTensorHandle k, AtenTensorHandle v,
    AtenTensorHandle offsets, AtenTensorHandle cuda_offsets, AtenTensorHandle blocks,
    double scale, AtenTensorHandle* output)"""
PROJECTION_GEMV_C_SHIM = """AOTITorchError aoti_torch_cuda_projection_gemv(
    AtenTensorHandle x, AtenTensorHandle weight, AtenTensorHandle* output)"""
NORM_ROPE_C_SHIM = """AOTITorchError aoti_torch_cuda_qk_norm_rope_append(
    AtenTensorHandle q, AtenTensorHandle key, AtenTensorHandle value,
    AtenTensorHandle q_weight, AtenTensorHandle k_weight, double eps,
    AtenTensorHandle cos, AtenTensorHandle sin, AtenTensorHandle positions,
    AtenTensorHandle cu_query, AtenTensorHandle cache_key, AtenTensorHandle cache_value,
    AtenTensorHandle* output)"""
MODELS = ("qwen3", "qwen35")
_loaded = None


def require(condition, message):
    """Raise ValueError(message) unless condition holds (a check that survives ``python -O``)."""
    if not condition:
        raise ValueError(message)


def default_build_dir(model):
    """One library serves every model family (reference: artifacts.py:11-13)."""
    require(model in MODELS, f"Unknown model {model!r}; expected one of {MODELS}")
    return ROOT / "lib"


def cache_extent(valid_length):
    """CPU uint8 tensor of length valid_length + 1 that carries L to flash_attention.

    The operator reads nothing but its length.  The extra element keeps the
    length at 2 or more, so AOTInductor never specialises it as a size-one
    dimension.
    """
    import torch

    return torch.empty(valid_length + 1, dtype=torch.uint8)


def batched_attention_metadata(kv_lengths, query_lengths, device):
    """Cumulative query/KV lengths for one step, shared by every layer.

    Returns (CPU offsets [2,B+1] int32, their device copy, device blocks [B,1]):
    row 0 holds cumulative real-query counts, row 1 cumulative KV lengths.  The
    CPU copy drives scheduling without a device readback; the device copy drives
    the KV append.  Reference: compiler/common/attention.py:27-40.
    """
    import torch

    lengths = torch.stack((query_lengths, kv_lengths))
    offsets = torch.cat(
        (torch.zeros((2, 1), dtype=torch.int32), lengths.cumsum(1, dtype=torch.int32)), dim=1
    )
    blocks = torch.arange(kv_lengths.shape[0], device=device, dtype=torch.int32)[:, None]
    if torch.device(device).type == "cuda" and not _tracing():
        # Eager serving: a pinned source lets the copy queue on the current
        # stream without blocking the host, and makes it a capturable graph
        # node.  A traced graph (torch.export, torch.compile) records the plain
        # copy instead: fake tensors have no pinned storage.
        offsets = offsets.pin_memory()
        return offsets, offsets.to(device, non_blocking=True), blocks
    return offsets, offsets.to(device), blocks


def _tracing():
    """True while torch.export / torch.compile trace the caller, or under a fake mode."""
    import torch

    if torch.compiler.is_compiling():
        return True
    from torch._guards import detect_fake_mode

    return detect_fake_mode() is not None


def load_attention_ops(library=None, *, model=None):
    """Load the native operators once per process and register their fakes.

    Selection order as in the reference (attention.py:43-58): explicit
    ``library``, then ``XINFER_ATTENTION_OPS_LIBRARY``, then the model's default
    build.  A missing library raises FileNotFoundError; a second, different
    library in one process raises ValueError.
    """
    global _loaded
    if library is None and _loaded is not None:
        return
    selected = library or os.environ.get("XINFER_ATTENTION_OPS_LIBRARY")
    if not selected:
        if model is None:
            raise ValueError("Select a model to locate its default native attention library")
        selected = default_build_dir(model) / ATTENTION_LIBRARY
    library = Path(selected).resolve()
    if _loaded is not None:
        if _loaded != library:
            raise ValueError("Cannot load two different attention libraries in one Python process")
        return
    if not library.is_file():
        raise FileNotFoundError(f"Build the native attention library first: {library}")
    import torch

    torch.ops.load_library(str(library))

    @torch.library.register_fake("xinfer::flash_attention")
    def fake(q, k, v, kv_extent, scale):
        # Shapes, dtypes and devices only: the valid length (kv_extent's
        # length) is validated by the native operator, and the output takes
        # q's shape and dtype.
        torch._check(q.dim() == 4 and k.dim() == 4 and v.dim() == 4)
        torch._check(q.shape[0] > 0)
        torch._check(q.shape[1] > 0)
        torch._check(k.shape[1] > 0)
        torch._check(q.shape[1] % k.shape[1] == 0)
        torch._check(q.shape[3] >= 8)
        torch._check(q.shape[3] <= 256)
        torch._check(q.shape[3] % 8 == 0)
        torch._check(q.shape[2] >= 1)
        torch._check(q.shape[2] <= 512)
        torch._check(k.shape[2] > 0)
        torch._check(k.shape == (q.shape[0], k.shape[1], k.shape[2], q.shape[3]))
        torch._check(v.shape == k.shape)
        torch._check(q.dtype == k.dtype == v.dtype == torch.bfloat16)
        torch._check(q.device.type == "cuda" and k.device == q.device and v.device == q.device)
        torch._check(kv_extent.device.type == "cpu" and kv_extent.dtype == torch.uint8)
        torch._check(kv_extent.dim() == 1)
        return q.new_empty(q.shape)

    if hasattr(torch.ops.xinfer, "batched_flash_attention"):

        @torch.library.register_fake("xinfer::batched_flash_attention")
        def fake_batched(q, k, v, offsets, cuda_offsets, blocks, scale):
            torch._check(offsets.device.type == "cpu" and offsets.dtype == torch.int32)
            torch._check(offsets.shape == (2, q.shape[0] + 1))
            torch._check(cuda_offsets.shape == offsets.shape and cuda_offsets.device == q.device)
            torch._check(blocks.shape == (q.shape[0], 1) and blocks.device == q.device)
            return fake(q, k, v, torch.empty(2, dtype=torch.uint8), scale)

    if hasattr(torch.ops.xinfer, "batched_flash_attention_bthd"):

        @torch.library.register_fake("xinfer::batched_flash_attention_bthd")
        def fake_batched_bthd(q, k, v, offsets, cuda_offsets, blocks, scale):
            out = fake_batched(q, k, v, offsets, cuda_offsets, blocks, scale)
            return out.new_empty((q.shape[0], q.shape[2], q.shape[1], q.shape[3]))

    if hasattr(torch.ops.xinfer, "batched_flash_attention_graph"):

        @torch.library.register_fake("xinfer::batched_flash_attention_graph")
        def fake_batched_graph(q, k, v, offsets, cuda_offsets, blocks, scale):
            torch._check(q.shape[2] * (q.shape[1] // k.shape[1]) <= 8)
            return fake_batched(q, k, v, offsets, cuda_offsets, blocks, scale)

    if hasattr(torch.ops.xinfer, "append_kv_batched"):

        @torch.library.register_fake("xinfer::append_kv_batched")
        def fake_append(key, value, positions, cu_query, cache_key, cache_value):
            # The reference's only contract check (kv_cache.py:54-55).
            torch._check(cache_key.is_contiguous() and cache_value.is_contiguous())
            return None

    if hasattr(torch.ops.xinfer, "projection_gemv"):

        @torch.library.register_fake("xinfer::projection_gemv")
        def fake_projection(x, weight):
            torch._check(weight.dim() == 2 and x.dim() >= 2 and x.shape[-1] == weight.shape[1])
            return x.new_empty((*x.shape[:-1], weight.shape[0]))

    if hasattr(torch.ops.xinfer, "qk_norm_rope_append"):

        @torch.library.register_fake("xinfer::qk_norm_rope_append")
        def fake_norm_rope(q, key, value, q_weight, k_weight, eps, cos, sin, positions, cu_query,
                           cache_key, cache_value):
            torch._check(q.dim() == 4 and key.dim() == 4 and value.shape == key.shape)
            torch._check(key.shape[0] == q.shape[0] and key.shape[1] == q.shape[1])
            torch._check(key.shape[3] == q.shape[3])
            torch._check(cos.shape == (q.shape[0], q.shape[1], q.shape[3]) and sin.shape == cos.shape)
            torch._check(q_weight.shape == (q.shape[3],) and k_weight.shape == q_weight.shape)
            torch._check(cache_key.is_contiguous() and cache_value.is_contiguous())
            return q.new_empty((q.shape[0], q.shape[2], q.shape[1], q.shape[3]))

    _loaded = library


def attention_library():
    """Path of the library loaded in this process, which export embeds in its packages."""
    require(_loaded is not None, "Load the native attention library before export")
    return _loaded


def attention_c_shims():
    """Inductor's call declarations for the registered operators.

    The reference maps the two attention operators (attention.py:105-112); the
    native append needs its own entry because it is no longer a Triton op, and
    so do the fused norm/rope/append step, the [B,T,Hq,D]-output variant and
    the native projection GEMV (a Triton op in the reference).
    """
    import torch

    return {
        torch.ops.xinfer.flash_attention.default: [ATTENTION_C_SHIM],
        torch.ops.xinfer.batched_flash_attention.default: [BATCHED_ATTENTION_C_SHIM],
        torch.ops.xinfer.append_kv_batched.default: [APPEND_KV_C_SHIM],
        torch.ops.xinfer.qk_norm_rope_append.default: [NORM_ROPE_C_SHIM],
        torch.ops.xinfer.batched_flash_attention_bthd.default: [BATCHED_BTHD_C_SHIM],
        torch.ops.xinfer.projection_gemv.default: [PROJECTION_GEMV_C_SHIM],
    }
