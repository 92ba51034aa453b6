"""The allocation-free batched attention entry point through the C ABI.

xinfer_batched_flash_attention_noalloc runs the same plan and kernels as
xinfer_batched_flash_attention, with the split records in the library's
static device scratch instead of a caller's workspace.  Three calls in a row
-- a 512-token prefill chunk whose records fill half of the scratch, a
smaller ragged decode batch, and a short-row decode batch whose splits the
decode launch merges itself, with its arrival counters in the scratch -- must
each equal the workspace entry point bit for bit (each call finds the earlier
calls' records in the scratch and must not depend on them), and stay within
the oracle gates.  A plan beyond
the scratch is refused before any launch.  In a fresh process, the first
call (which looks up the scratch's device address) is made while a HIP graph
is being captured; every replay of that graph must equal the workspace entry
point bit for bit.
"""

import ctypes
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from attn_helpers import MAX_ABS, MEAN_ABS, log
from oracle import attention as oracle

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


class View4(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("size", ctypes.c_int64 * 4), ("stride", ctypes.c_int64 * 4)]


def view(t):
    return View4(t.data_ptr(), (ctypes.c_int64 * 4)(*t.shape), (ctypes.c_int64 * 4)(*t.stride()))


@pytest.fixture(scope="module")
def capi(library_path):
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a visible AMD GPU")
    lib = ctypes.CDLL(str(library_path))
    lib.xinfer_status_string.restype = ctypes.c_char_p
    lib.xinfer_batched_flash_attention_workspace_size.restype = ctypes.c_size_t
    return lib


def host_offsets(counts, lengths):
    offsets = [0]
    for count in counts:
        offsets.append(offsets[-1] + count)
    offsets.append(0)
    for length in lengths:
        offsets.append(offsets[-1] + length)
    return (ctypes.c_int32 * len(offsets))(*offsets)


def case(seed, batch, heads, kv_heads, dim, capacity, counts, lengths):
    generator = torch.Generator().manual_seed(seed)

    def draw(*shape):
        return torch.randn(*shape, generator=generator).to(torch.bfloat16).cuda()

    q = draw(batch, max(counts), heads, dim).transpose(1, 2)
    return q, draw(batch, kv_heads, capacity, dim), draw(batch, kv_heads, capacity, dim)


def run_both(capi, q, k, v, counts, lengths, scale):
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    qv, kv, vv = view(q), view(k), view(v)
    host = host_offsets(counts, lengths)
    size = capi.xinfer_batched_flash_attention_workspace_size(ctypes.byref(qv), ctypes.byref(kv), host)
    assert 0 < size <= SCRATCH_BYTES
    out = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device="cuda")
    status = capi.xinfer_batched_flash_attention_noalloc(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), host,
                                                         None, ctypes.c_int64(0), ctypes.c_double(scale),
                                                         ctypes.c_void_p(out.data_ptr()), stream)
    assert status == 0, capi.xinfer_status_string(status)
    workspace = torch.empty(size, dtype=torch.uint8, device="cuda")
    expected = torch.empty(q.shape, dtype=torch.bfloat16, device="cuda")
    status = capi.xinfer_batched_flash_attention(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), host,
                                                 None, ctypes.c_int64(0), ctypes.c_double(scale),
                                                 ctypes.c_void_p(expected.data_ptr()),
                                                 ctypes.c_void_p(workspace.data_ptr()), ctypes.c_size_t(size), stream)
    assert status == 0, capi.xinfer_status_string(status)
    torch.cuda.synchronize()
    return out, expected, size


def check_oracle(out, q, k, v, counts, lengths, scale):
    reference = oracle.attention(*(x.float().cpu().numpy().astype(np.float64) for x in (q, k, v)),
                                 counts, lengths, scale)
    delta = np.abs(out.float().cpu().numpy() - reference)
    assert delta.max() <= MAX_ABS
    for r, count in enumerate(counts):
        assert not out[r, :, count:].any()
        if count:
            assert delta[r, :, :count].mean() <= MEAN_ABS


@torch.inference_mode()
def test_noalloc_equals_the_workspace_entry_point_on_three_calls(capi):
    # First call: a 512-token chunk at offset 1536 (records fill half the scratch).
    counts, lengths = [512], [2048]
    log(f"no-alloc call 1: prefill counts={counts} lengths={lengths}")
    q, k, v = case(5, 1, 16, 8, 128, 4096, counts, lengths)
    out, expected, size = run_both(capi, q, k, v, counts, lengths, 128**-0.5)
    assert size > SCRATCH_BYTES // 4
    assert torch.equal(out.view(torch.int16), expected.view(torch.int16))
    check_oracle(out, q, k, v, counts, lengths, 128**-0.5)
    # Second call: a smaller ragged decode batch, over the first call's records.
    counts, lengths = [1, 1, 1, 0], [13312, 386, 9459, 20]
    log(f"no-alloc call 2: decode counts={counts} lengths={lengths}")
    q, k, v = case(6, 4, 16, 8, 128, 16384, counts, lengths)
    out2, expected2, size2 = run_both(capi, q, k, v, counts, lengths, 128**-0.5)
    assert 0 < size2 < size
    assert torch.equal(out2.view(torch.int16), expected2.view(torch.int16))
    check_oracle(out2, q, k, v, counts, lengths, 128**-0.5)
    # Third call: a short-row decode batch whose splits the decode launch
    # merges itself (arrival counters in the scratch, past the records).
    counts, lengths = [1, 1, 1], [1024, 700, 900]
    log(f"no-alloc call 3: decode counts={counts} lengths={lengths}")
    q, k, v = case(8, 3, 16, 8, 128, 2048, counts, lengths)
    out3, expected3, size3 = run_both(capi, q, k, v, counts, lengths, 128**-0.5)
    assert 0 < size3 < size2
    assert torch.equal(out3.view(torch.int16), expected3.view(torch.int16))
    check_oracle(out3, q, k, v, counts, lengths, 128**-0.5)


@torch.inference_mode()
def test_noalloc_refuses_plans_beyond_its_scratch(capi):
    counts = [356, 138, 422, 459, 325, 298, 113, 124]
    lengths = [14244, 13896, 2059, 4214, 12262, 14086, 12837, 9315]
    log("no-alloc oversize plan")
    q = torch.zeros(8, 16, 512, 256, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(8, 4, 16384, 256, dtype=torch.bfloat16, device="cuda")
    out = torch.full(q.shape, 7.0, dtype=torch.bfloat16, device="cuda")
    qv, kv = view(q), view(k)
    status = capi.xinfer_batched_flash_attention_noalloc(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(kv), host_offsets(counts, lengths), None, ctypes.c_int64(0),
        ctypes.c_double(1 / 16), ctypes.c_void_p(out.data_ptr()),
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert status == 17, capi.xinfer_status_string(status)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was launched


# Run in a fresh process, so that the entry point's first call -- the one that
# looks up the scratch's device address -- happens inside the capture.
CAPTURE_CHILD = r"""
import ctypes, sys
import torch
sys.path.insert(0, sys.argv[2])
from test_zz_no_alloc import host_offsets, view, case

lib = ctypes.CDLL(sys.argv[1])
lib.xinfer_status_string.restype = ctypes.c_char_p
lib.xinfer_batched_flash_attention_workspace_size.restype = ctypes.c_size_t
counts, lengths = [1, 1, 0, 1, 1, 1, 1, 1], [13312, 2162, 386, 9459, 1399, 3852, 55, 182]
q, k, v = case(7, 8, 16, 8, 128, 16384, counts, lengths)
qv, kv, vv = view(q), view(k), view(v)
host = host_offsets(counts, lengths)
scale = ctypes.c_double(128 ** -0.5)
size = lib.xinfer_batched_flash_attention_workspace_size(ctypes.byref(qv), ctypes.byref(kv), host)
assert size > 0
side = torch.cuda.Stream()
side.wait_stream(torch.cuda.current_stream())
with torch.cuda.stream(side):
    # The workspace entry point first, eagerly: the expected result (and the
    # kernels' first launches) before any capture.
    workspace = torch.empty(size, dtype=torch.uint8, device="cuda")
    expected = torch.empty(q.shape, dtype=torch.bfloat16, device="cuda")
    status = lib.xinfer_batched_flash_attention(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), host, None,
                                                ctypes.c_int64(0), scale, ctypes.c_void_p(expected.data_ptr()),
                                                ctypes.c_void_p(workspace.data_ptr()), ctypes.c_size_t(size),
                                                ctypes.c_void_p(side.cuda_stream))
    assert status == 0, lib.xinfer_status_string(status)
    out = torch.full(q.shape, float("nan"), dtype=torch.bfloat16, device="cuda")
torch.cuda.current_stream().wait_stream(side)
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    status = lib.xinfer_batched_flash_attention_noalloc(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(vv), host, None, ctypes.c_int64(0), scale,
        ctypes.c_void_p(out.data_ptr()), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
assert status == 0, lib.xinfer_status_string(status)
torch.cuda.synchronize()
for replay in range(3):
    out.fill_(float("nan"))
    graph.replay()
    _ = torch.randn(1 << 20, device="cuda").sum()  # other eager work between replays
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), replay
print("noalloc capture ok", flush=True)
"""


@torch.inference_mode()
def test_noalloc_first_call_inside_graph_capture(library_path):
    log("no-alloc: first call inside a graph capture (fresh process)")
    tests = Path(__file__).resolve().parent
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(filter(None, [str(tests.parent), os.environ.get("PYTHONPATH")])))
    result = subprocess.run([sys.executable, "-c", CAPTURE_CHILD, str(library_path), str(tests)],
                            capture_output=True, text=True, timeout=300, env=env)
    assert result.returncode == 0, result.stdout[-2000:] + result.stderr[-4000:]
    assert "noalloc capture ok" in result.stdout
