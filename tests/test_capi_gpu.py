"""The C ABI called directly through ctypes, as a non-torch host would bind it.

Device memory comes from torch (plumbing only); every compute call goes through
the extern "C" entry points of include/xinfer_attention.h and must agree bit for
bit with the torch operators built on the same kernels, and with the oracle.
"""

import ctypes

import numpy as np
import pytest
import torch

from attn_helpers import MAX_ABS, MEAN_ABS, log
from oracle import attention as oracle
from xinfer_amd.attention import batched_attention_metadata

pytestmark = pytest.mark.gpu


class View4(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("size", ctypes.c_int64 * 4), ("stride", ctypes.c_int64 * 4)]


def view(t):
    return View4(t.data_ptr(), (ctypes.c_int64 * 4)(*t.shape), (ctypes.c_int64 * 4)(*t.stride()))


@pytest.fixture(scope="module")
def capi(gpu_ops, library_path):
    lib = ctypes.CDLL(str(library_path))
    lib.xinfer_status_string.restype = ctypes.c_char_p
    lib.xinfer_batched_flash_attention_workspace_size.restype = ctypes.c_size_t
    lib.xinfer_flash_attention_workspace_size.restype = ctypes.c_size_t
    return lib


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@torch.inference_mode()
def test_batched_through_c_abi(capi, gpu_ops):
    torch.manual_seed(77)
    batch, heads, kv_heads, dim, capacity = 4, 16, 4, 256, 2048
    counts, lengths = [1, 300, 0, 2], [1800, 700, 9, 40]
    log(f"C ABI batched counts={counts} lengths={lengths}")
    q = torch.randn(batch, max(counts), heads, dim, device="cuda", dtype=torch.bfloat16).transpose(1, 2)
    k = torch.randn(batch, kv_heads, capacity, dim, device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    host, cu, blocks = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    qv, kv, vv = view(q), view(k), view(v)
    offsets = host.contiguous()
    host_ptr = ctypes.cast(offsets.data_ptr(), ctypes.POINTER(ctypes.c_int32))
    size = capi.xinfer_batched_flash_attention_workspace_size(ctypes.byref(qv), ctypes.byref(kv), host_ptr)
    workspace = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty(q.shape, dtype=torch.bfloat16, device="cuda")
    status = capi.xinfer_batched_flash_attention(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), host_ptr, None, ctypes.c_int64(0),
        ctypes.c_double(dim**-0.5), ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(workspace.data_ptr()),
        ctypes.c_size_t(size), stream())
    assert status == 0, capi.xinfer_status_string(status)
    if size:
        too_small = capi.xinfer_batched_flash_attention(
            ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), host_ptr, None, ctypes.c_int64(0),
            ctypes.c_double(dim**-0.5),
            ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(workspace.data_ptr()), ctypes.c_size_t(size - 1),
            stream())
        assert capi.xinfer_status_string(too_small).decode().startswith("Attention workspace")
    via_torch = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, dim**-0.5)
    assert torch.equal(out.view(torch.int16), via_torch.view(torch.int16))
    expected = oracle.attention(*(x.float().cpu().numpy().astype(np.float64) for x in (q, k, v)),
                                counts, lengths, dim**-0.5)
    delta = np.abs(out.float().cpu().numpy() - expected)
    assert delta.max() <= MAX_ABS
    for r, count in enumerate(counts):
        assert not out[r, :, count:].any()
        if count:
            assert delta[r, :, :count].mean() <= MEAN_ABS


@torch.inference_mode()
def test_flash_and_append_through_c_abi(capi, gpu_ops):
    torch.manual_seed(78)
    heads, kv_heads, dim, capacity, tokens, length = 16, 8, 128, 4096, 512, 2048
    log("C ABI flash + append")
    q = torch.randn(1, heads, tokens, dim, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(1, kv_heads, capacity, dim, device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    new_k = torch.randn(1, tokens, kv_heads, dim, device="cuda", dtype=torch.bfloat16).transpose(1, 2)
    new_v = torch.randn_like(new_k)
    positions = torch.arange(length - tokens, length, device="cuda")[None]
    cu = torch.tensor([0, tokens], dtype=torch.int32, device="cuda")
    expected_k, expected_v = k.clone(), v.clone()
    expected_k[:, :, length - tokens : length] = new_k
    expected_v[:, :, length - tokens : length] = new_v
    status = capi.xinfer_append_kv_batched(
        ctypes.byref(view(new_k)), ctypes.byref(view(new_v)), ctypes.c_void_p(positions.data_ptr()),
        ctypes.c_int64(positions.stride(0)), ctypes.c_int64(positions.stride(1)), ctypes.c_void_p(cu.data_ptr()),
        ctypes.byref(view(k)), ctypes.byref(view(v)), stream())
    assert status == 0, capi.xinfer_status_string(status)
    assert torch.equal(k, expected_k) and torch.equal(v, expected_v)
    qv, kv, vv = view(q), view(k), view(v)
    size = capi.xinfer_flash_attention_workspace_size(ctypes.byref(qv), ctypes.byref(kv), ctypes.c_int64(length))
    workspace = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    status = capi.xinfer_flash_attention(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), ctypes.c_int64(length), ctypes.c_double(dim**-0.5),
        ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(workspace.data_ptr()), ctypes.c_size_t(size), stream())
    assert status == 0, capi.xinfer_status_string(status)
    from xinfer_amd.attention import cache_extent

    via_torch = gpu_ops.flash_attention(q, k, v, cache_extent(length), dim**-0.5)
    assert torch.equal(out.view(torch.int16), via_torch.view(torch.int16))


@torch.inference_mode()
def test_split_merge_survives_garbage_and_reused_workspace(capi, gpu_ops):
    """Split rows write partial records into the caller's workspace and a
    merge launch folds them.  A workspace full of arbitrary bytes, then the
    same workspace reused by later calls on other inputs, must still give the
    torch results: no record is read before it is written."""
    torch.manual_seed(79)
    batch, heads, kv_heads, dim, capacity = 3, 16, 8, 128, 16384
    counts, lengths = [1, 200, 1], [13000, 5000, 3000]
    log(f"C ABI split merge counts={counts} lengths={lengths}")
    host, cu, blocks = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    offsets = host.contiguous()
    host_ptr = ctypes.cast(offsets.data_ptr(), ctypes.POINTER(ctypes.c_int32))
    k = torch.randn(batch, kv_heads, capacity, dim, device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    q0 = torch.randn(batch, heads, max(counts), dim, device="cuda", dtype=torch.bfloat16)
    size = capi.xinfer_batched_flash_attention_workspace_size(
        ctypes.byref(view(q0)), ctypes.byref(view(k)), host_ptr)
    assert size > 0
    for fill in ("ones", "random", "reuse", "reuse"):
        q = torch.randn_like(q0)
        if fill == "ones":
            workspace = torch.full((size,), 0xFF, dtype=torch.uint8, device="cuda")
        elif fill == "random":
            workspace = torch.randint(0, 256, (size,), dtype=torch.uint8, device="cuda")
        out = torch.empty_like(q)
        status = capi.xinfer_batched_flash_attention(
            ctypes.byref(view(q)), ctypes.byref(view(k)), ctypes.byref(view(v)), host_ptr, None, ctypes.c_int64(0),
            ctypes.c_double(dim**-0.5), ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(workspace.data_ptr()),
            ctypes.c_size_t(size), stream())
        assert status == 0, capi.xinfer_status_string(status)
        via_torch = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, dim**-0.5)
        assert torch.equal(out.view(torch.int16), via_torch.view(torch.int16)), fill


@torch.inference_mode()
def test_split_merge_in_graph_replays(gpu_ops):
    """A captured call with split records and a merge launch replays exactly:
    every replay, on new inputs copied into the captured buffers, matches an
    eager call bit for bit."""
    torch.manual_seed(80)
    batch, heads, kv_heads, dim, capacity = 2, 16, 8, 128, 8192
    counts, lengths = [1, 512], [8000, 2048]
    log(f"graph replay split merge counts={counts} lengths={lengths}")
    host, cu, blocks = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    q = torch.randn(batch, heads, max(counts), dim, device="cuda", dtype=torch.bfloat16)
    k = torch.randn(batch, kv_heads, capacity, dim, device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, dim**-0.5)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, dim**-0.5)
    for replay in range(4):
        q.copy_(torch.randn_like(q))
        k[:, :, :64].copy_(torch.randn_like(k[:, :, :64]))
        graph.replay()
        torch.cuda.synchronize()
        eager = gpu_ops.batched_flash_attention(q, k, v, host, cu, blocks, dim**-0.5)
        torch.cuda.synchronize()
        assert torch.equal(captured.view(torch.int16), eager.view(torch.int16)), replay


@torch.inference_mode()
def test_fused_step_in_graph_replays(gpu_ops):
    """The serving step with the optional operators -- fused norm/rope/append,
    then attention with [B,T,Hq,D] output -- captured once and replayed on new
    projections: every replay matches an eager step bit for bit (output and
    both caches), with eager work in between.  The per-step metadata is built
    before capture, as a serving loop keeps it in persistent buffers."""
    from xinfer_amd.norm_rope import qk_norm_rope_append

    torch.manual_seed(81)
    batch, tokens, heads, kv_heads, dim, capacity = 4, 1, 16, 8, 128, 4096
    prefixes = [3000, 17, 900, 4000]
    counts = [1, 1, 0, 1]
    lengths = [p + c for p, c in zip(prefixes, counts)]
    options = dict(device="cuda", dtype=torch.bfloat16)
    q = torch.randn(batch, tokens, heads, dim, **options)
    k = torch.randn(batch, tokens, kv_heads, dim, **options)
    v = torch.randn_like(k)
    weights = [1 + 0.1 * torch.randn(dim, **options) for _ in range(2)]
    angle = torch.rand(batch, tokens, dim, device="cuda")
    cos, sin = angle.cos().to(torch.bfloat16), angle.sin().to(torch.bfloat16)
    positions = torch.tensor(prefixes, device="cuda")[:, None]
    caches = [torch.randn(batch, kv_heads, capacity, dim, **options) for _ in range(2)]
    base = [c.clone() for c in caches]
    host, cu, blocks = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")

    def step():
        qr = qk_norm_rope_append(q, k, v, weights[0], weights[1], 1e-6, cos, sin, positions, cu[0], *caches)
        return gpu_ops.batched_flash_attention_bthd(qr, caches[0], caches[1], host, cu, blocks, dim**-0.5)

    step()  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for replay in range(3):
        for c, b in zip(caches, base):
            c.copy_(b)
        q.copy_(torch.randn_like(q))
        k.copy_(torch.randn_like(k))
        graph.replay()
        torch.cuda.synchronize()
        replayed = [captured.clone()] + [c.clone() for c in caches]
        for c, b in zip(caches, base):
            c.copy_(b)
        eager = step()
        torch.cuda.synchronize()
        assert torch.equal(replayed[0].view(torch.int16), eager.view(torch.int16)), replay
        assert all(torch.equal(a, b) for a, b in zip(replayed[1:], caches)), replay


@torch.inference_mode()
def test_page_table_through_c_abi(capi, gpu_ops):
    """The C entry points with a page table (device pointer and row stride):
    the workspace entry point and the allocation-free one give the torch
    operator's bits for a permuted table viewed with row stride 2."""
    counts, lengths, capacity, dim = [1, 40, 0, 1], [700, 300, 5, 1024], 1024, 128
    log(f"C ABI page table: counts={counts} lengths={lengths} C={capacity}")
    generator = torch.Generator().manual_seed(5)
    q = torch.randn(4, 16, 40, dim, generator=generator).to(torch.bfloat16).cuda()
    k = torch.randn(4, 8, capacity, dim, generator=generator).to(torch.bfloat16).cuda()
    v = torch.randn(4, 8, capacity, dim, generator=generator).to(torch.bfloat16).cuda()
    host, cu, _ = batched_attention_metadata(
        torch.tensor(lengths, dtype=torch.int32), torch.tensor(counts, dtype=torch.int32), "cuda")
    table = torch.tensor([[2, 7], [0, 7], [3, 7], [1, 7]], dtype=torch.int32).cuda()[:, :1]
    assert table.stride(0) == 2
    expected = gpu_ops.batched_flash_attention(q, k, v, host, cu, table, dim**-0.5)
    qv, kv, vv = view(q), view(k), view(v)
    offsets = host.contiguous()
    host_ptr = ctypes.cast(offsets.data_ptr(), ctypes.POINTER(ctypes.c_int32))
    pages, stride_ = ctypes.c_void_p(table.data_ptr()), ctypes.c_int64(table.stride(0))
    size = capi.xinfer_batched_flash_attention_workspace_size(ctypes.byref(qv), ctypes.byref(kv), host_ptr)
    workspace = torch.empty(max(size, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty_like(q)
    status = capi.xinfer_batched_flash_attention(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), host_ptr, pages, stride_, ctypes.c_double(dim**-0.5),
        ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(workspace.data_ptr()), ctypes.c_size_t(size), stream())
    assert status == 0, capi.xinfer_status_string(status)
    free = torch.empty_like(q)
    status = capi.xinfer_batched_flash_attention_noalloc(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), host_ptr, pages, stride_, ctypes.c_double(dim**-0.5),
        ctypes.c_void_p(free.data_ptr()), stream())
    assert status == 0, capi.xinfer_status_string(status)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), expected.view(torch.int16))
    assert torch.equal(free.view(torch.int16), expected.view(torch.int16))
    moved = gpu_ops.batched_flash_attention(q, k[[2, 0, 3, 1]].contiguous(), v[[2, 0, 3, 1]].contiguous(), host, cu,
                                            torch.arange(4, dtype=torch.int32, device="cuda").view(4, 1), dim**-0.5)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), moved.view(torch.int16))
