"""CPU checks of libxinfer_attention_ops.so: exports, messages, validation, schemas, fakes.

Nothing here launches a kernel: every C-ABI call below fails validation (or only
queries a workspace size) before any HIP call, so these run without a GPU.
"""

import ctypes
from pathlib import Path
import re

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))

# Reference operator messages (compiler/common/kernels/attention.cpp).
REFERENCE_MESSAGES = {
    1: "Invalid Q/K/V shapes",                                              # :17-19
    2: "Unsupported Q shape",                                               # :90-91
    3: "Expected matching full-capacity K/V inputs [batch,kv_heads,capacity,head_dim]",  # :92-94
    4: "Query heads must be a positive multiple of KV heads",               # :95-96
    5: "Flash head dimension must be a multiple of 8 in 8..256",            # :97-98
    6: "Invalid valid-prefix length",                                       # :102
    7: "Attention scale must be finite and positive",                       # :103
    8: "Cumulative lengths must start at zero",                             # :35
    9: "Invalid query/KV lengths",                                          # :43-45
}
REFERENCE_SCHEMAS = {
    # attention.cpp:129-134 and the triton_op schema inferred from kv_cache.py:45-52.
    "batched_flash_attention": "xinfer::batched_flash_attention(Tensor q, Tensor k, Tensor v, Tensor offsets, "
    "Tensor cuda_offsets, Tensor blocks, float scale) -> Tensor",
    "flash_attention": "xinfer::flash_attention(Tensor q, Tensor k, Tensor v, Tensor kv_extent, float scale) -> Tensor",
    "append_kv_batched": "xinfer::append_kv_batched(Tensor key, Tensor value, Tensor positions, Tensor cu_query, "
    "Tensor(a4!) cache_key, Tensor(a5!) cache_value) -> ()",
}


class View4(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("size", ctypes.c_int64 * 4), ("stride", ctypes.c_int64 * 4)]


def view(sizes, strides=None, data=1 << 20):
    if strides is None:
        strides = [sizes[1] * sizes[2] * sizes[3], sizes[2] * sizes[3], sizes[3], 1]
    return View4(data, (ctypes.c_int64 * 4)(*sizes), (ctypes.c_int64 * 4)(*strides))


def declared_functions():
    names = []
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        text = re.sub(r"^\s*#[^\n]*", "", text, flags=re.M)  # preprocessor lines
        for match in re.finditer(r"\b([A-Za-z_]\w*)\s*\([^;{}]*\)\s*;", text):
            names.append(match.group(1))
    return names


@pytest.fixture(scope="module")
def lib(library_path):
    torch.ops.load_library(str(library_path))  # resolves libtorch for the shim symbols
    handle = ctypes.CDLL(str(library_path))
    handle.xinfer_status_string.restype = ctypes.c_char_p
    handle.xinfer_flash_attention_workspace_size.restype = ctypes.c_size_t
    handle.xinfer_batched_flash_attention_workspace_size.restype = ctypes.c_size_t
    return handle


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert {"xinfer_flash_attention", "xinfer_batched_flash_attention", "xinfer_append_kv_batched",
            "xinfer_qk_norm_rope_append", "xinfer_batched_flash_attention_out", "xinfer_projection_gemv",
            "aoti_torch_cuda_projection_gemv", "aoti_torch_cuda_flash_attention",
            "aoti_torch_cuda_batched_flash_attention", "aoti_torch_cuda_append_kv_batched",
            "aoti_torch_cuda_qk_norm_rope_append", "xinfer_batched_flash_attention_noalloc",
            "xinfer_batched_flash_attention_graph"} <= set(names)
    for name in names:
        assert hasattr(lib, name), f"{name} is declared in include/ but not exported"


def test_status_messages_match_the_reference(lib):
    for code, message in REFERENCE_MESSAGES.items():
        assert lib.xinfer_status_string(code).decode() == message


def flash(lib, q, k, length, scale=0.1):
    return lib.xinfer_flash_attention(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k),
                                      ctypes.c_int64(length), ctypes.c_double(scale),
                                      ctypes.c_void_p(1 << 20), None, ctypes.c_size_t(0), None)


def test_flash_validation_order_and_codes(lib):
    q, k = view([1, 16, 2, 128]), view([1, 8, 64, 128])
    assert flash(lib, view([1, 16, 513, 128]), k, 600) == 2
    assert flash(lib, view([0, 16, 2, 128]), view([0, 8, 64, 128]), 5) == 2
    assert flash(lib, q, view([2, 8, 64, 128]), 5) == 3
    assert flash(lib, view([1, 12, 2, 128]), k, 5) == 4
    assert flash(lib, view([1, 16, 2, 127]), view([1, 8, 64, 127]), 5) == 5
    assert flash(lib, view([1, 16, 2, 264]), view([1, 8, 64, 264]), 5) == 5
    for length in (0, 1, 65):
        assert flash(lib, q, k, length) == 6
    assert flash(lib, q, k, 5, scale=-1.0) == 7
    assert flash(lib, q, k, 5, scale=float("inf")) == 7
    strided = view([1, 16, 2, 128], [4096 * 2, 256 * 2, 2048 * 2, 2])
    assert flash(lib, strided, k, 5) == 11


ARGUMENT = 14  # XINFER_ERR_ARGUMENT


def batched(lib, q, k, offsets, scale=0.1, blocks=None, stride=0):
    host = (ctypes.c_int32 * len(offsets))(*offsets)
    return lib.xinfer_batched_flash_attention(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), host,
                                              blocks, ctypes.c_int64(stride), ctypes.c_double(scale),
                                              ctypes.c_void_p(1 << 20), None, ctypes.c_size_t(0), None)


def test_batched_validation_codes(lib):
    q, k = view([2, 16, 4, 128]), view([2, 8, 64, 128])
    assert batched(lib, q, view([3, 8, 64, 128]), [0, 1, 2, 0, 5, 9]) == 1
    assert batched(lib, q, k, [1, 1, 2, 0, 5, 9]) == 8
    assert batched(lib, q, k, [0, 5, 6, 0, 5, 9]) == 9   # count > T
    assert batched(lib, q, k, [0, 1, 2, 0, 0, 9]) == 9   # length < 1
    assert batched(lib, q, k, [0, 3, 4, 0, 2, 9]) == 9   # length < count
    assert batched(lib, q, k, [0, 1, 2, 0, 65, 70]) == 9  # length > capacity
    assert batched(lib, q, k, [0, 1, 2, 0, 5, 9], scale=0.0) == 7
    # A page table is a 4-byte aligned device pointer with a non-negative row stride.
    assert batched(lib, q, k, [0, 1, 2, 0, 5, 9], blocks=ctypes.c_void_p((1 << 21) + 2), stride=1) == ARGUMENT
    assert batched(lib, q, k, [0, 1, 2, 0, 5, 9], blocks=ctypes.c_void_p(1 << 21), stride=-1) == ARGUMENT


def norm_rope(lib, q, k, rope, cache, eps=1e-6, cu_query=1 << 21):
    return lib.xinfer_qk_norm_rope_append(
        ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), ctypes.c_void_p(1 << 22), ctypes.c_void_p(1 << 22),
        ctypes.c_double(eps), ctypes.byref(rope), ctypes.byref(rope), ctypes.c_void_p(1 << 23), ctypes.c_int64(4),
        ctypes.c_int64(1), ctypes.c_void_p(cu_query), ctypes.c_void_p(1 << 24), ctypes.byref(cache),
        ctypes.byref(cache), None)


def test_norm_rope_validation_codes(lib):
    """Every rejected input returns before any launch (no device is touched)."""
    q, k, rope, cache = view([2, 16, 4, 128]), view([2, 8, 4, 128]), view([2, 1, 4, 128]), view([2, 8, 64, 128])
    assert lib.xinfer_status_string(15).decode().startswith("Expected q [B,Hq,T,D]")
    assert lib.xinfer_status_string(16).decode() == "RMSNorm epsilon must be finite and non-negative"
    assert norm_rope(lib, view([2, 16, 4, 96]), view([2, 8, 4, 96]), view([2, 1, 4, 96]), view([2, 8, 64, 96])) == 15
    assert norm_rope(lib, q, view([2, 8, 5, 128]), rope, cache) == 15
    assert norm_rope(lib, q, k, view([2, 2, 4, 128]), cache) == 15
    assert norm_rope(lib, q, k, rope, cache, eps=-1.0) == 16
    assert norm_rope(lib, q, k, rope, cache, eps=float("nan")) == 16
    assert norm_rope(lib, view([0, 16, 4, 128]), view([0, 8, 4, 128]), view([0, 1, 4, 128]), cache) == 0
    assert norm_rope(lib, q, k, rope, cache, cu_query=0) == 14
    assert norm_rope(lib, view([2, 16, 4, 128], data=(1 << 20) + 2), k, rope, cache) == 11
    assert norm_rope(lib, view([2, 16, 4, 128], [16 * 4 * 132, 4 * 132, 132, 1]), k, rope, cache) == 11
    assert norm_rope(lib, q, k, rope, view([2, 8, 64, 128], [8 * 64 * 128, 128, 8 * 128, 1])) == 12
    assert norm_rope(lib, q, k, rope, view([2, 4, 64, 128])) == 12


def test_output_view_validation_codes(lib):
    """xinfer_batched_flash_attention_out checks its output view before any launch."""
    q, k = view([2, 16, 4, 128]), view([2, 8, 64, 128])
    host = (ctypes.c_int32 * 6)(0, 1, 2, 0, 5, 9)

    def call(out):
        return lib.xinfer_batched_flash_attention_out(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), host,
                                                      None, ctypes.c_int64(0), ctypes.c_double(0.1), out, None,
                                                      ctypes.c_size_t(0), None)

    assert call(None) == 14
    assert call(ctypes.byref(view([2, 16, 5, 128]))) == 1
    assert call(ctypes.byref(view([2, 16, 4, 128], data=(1 << 20) + 8))) == 11
    assert call(ctypes.byref(view([2, 16, 4, 128], [4 * 16 * 128, 128, 16 * 128 + 4, 1]))) == 11
    assert call(ctypes.byref(view([2, 16, 4, 128], [4 * 16 * 256, 256, 16 * 256, 2]))) == 11


def test_projection_gemv_validation_codes(lib):
    """Rejected arguments return before any launch."""
    call = lambda x, w, out, n, k, dtype: lib.xinfer_projection_gemv(  # noqa: E731
        ctypes.c_void_p(x), ctypes.c_void_p(w), ctypes.c_void_p(out), ctypes.c_int64(n), ctypes.c_int64(k),
        ctypes.c_int(dtype), None)
    assert call(0, 1 << 20, 1 << 21, 4, 8, 0) == 14
    assert call(1 << 20, 1 << 20, 1 << 21, 0, 8, 0) == 14
    assert call(1 << 20, 1 << 20, 1 << 21, 4, -1, 1) == 14
    assert call(1 << 20, 1 << 20, 1 << 21, 4, 8, 2) == 14


def test_workspace_size_is_a_pure_host_query(lib):
    q, k = view([8, 16, 1, 128]), view([8, 8, 16384, 128])
    lengths = [13312, 2162, 386, 9459, 1399, 3852, 55, 182]
    offsets = [0, 1, 2, 3, 4, 5, 6, 7, 8, 0]
    for length in lengths:
        offsets.append(offsets[-1] + length)
    host = (ctypes.c_int32 * len(offsets))(*offsets)
    bytes_ = lib.xinfer_batched_flash_attention_workspace_size(ctypes.byref(q), ctypes.byref(k), host)
    assert bytes_ > 0
    # A workspace of that size that is not 16-byte aligned is refused before any launch.
    assert lib.xinfer_batched_flash_attention(ctypes.byref(q), ctypes.byref(k), ctypes.byref(k), host, None,
                                              ctypes.c_int64(0), ctypes.c_double(0.1), ctypes.c_void_p(1 << 20),
                                              ctypes.c_void_p((1 << 22) + 8), ctypes.c_size_t(bytes_), None) == 10
    assert lib.xinfer_status_string(10).decode() == (
        "Attention workspace is smaller than its size query or not 16-byte aligned")
    # One short row with one split needs no partial records.
    q1, k1 = view([1, 16, 1, 128]), view([1, 8, 4096, 128])
    assert lib.xinfer_flash_attention_workspace_size(ctypes.byref(q1), ctypes.byref(k1), ctypes.c_int64(100)) == 0


def test_noalloc_rejects_plans_beyond_its_scratch_before_any_launch(lib):
    """The allocation-free entry point validates like the workspace one and
    refuses a plan whose split records exceed its static scratch (32 MiB)
    with its own status, before any HIP call."""
    assert lib.xinfer_status_string(17).decode().startswith("Attention needs more split-record scratch")
    counts = [356, 138, 422, 459, 325, 298, 113, 124]
    lengths = [14244, 13896, 2059, 4214, 12262, 14086, 12837, 9315]
    q, k = view([8, 16, 512, 256]), view([8, 4, 16384, 256])
    offsets = [0]
    for count in counts:
        offsets.append(offsets[-1] + count)
    offsets.append(0)
    for length in lengths:
        offsets.append(offsets[-1] + length)
    host = (ctypes.c_int32 * len(offsets))(*offsets)
    assert lib.xinfer_batched_flash_attention_workspace_size(ctypes.byref(q), ctypes.byref(k), host) > 32 << 20

    def noalloc(qv, kv, offsets_, scale=1.0):
        return lib.xinfer_batched_flash_attention_noalloc(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(kv),
                                                          offsets_, None, ctypes.c_int64(0), ctypes.c_double(scale),
                                                          ctypes.c_void_p(1 << 20), None)

    assert noalloc(q, k, host) == 17
    # The checks of the workspace entry point come first, with its codes.
    assert noalloc(q, k, host, scale=float("nan")) == 7
    bad = (ctypes.c_int32 * len(offsets))(*([1] + offsets[1:]))
    assert noalloc(q, k, bad) == 8


def test_graph_mode_shapes_and_workspace(lib):
    """The graph-capture entry point plans from shapes alone: its workspace
    holds every row's records at capacity, and more than 64 rows are refused
    before any launch.  Decode items take four rounds of 128 keys (D = 128,
    two query vectors per KV head) when the capacity layout holds at least
    1536 one-round items and at most 2048 four-round ones, else one round.
    Prefill shapes (T * Hq/Hkv > 8) hold records for the most items the
    device plan can lay out: 2048 plus one per (row, kv head, query tile), or
    every such unit split 8 ways (C / 512 ways below 4096 keys), whichever
    is fewer, followed by the device-written prefill and merge arguments."""
    lib.xinfer_batched_flash_attention_graph_workspace_size.restype = ctypes.c_size_t

    def workspace(batch, capacity):
        q, k = view([batch, 16, 1, 128]), view([batch, 8, capacity, 128])
        return lib.xinfer_batched_flash_attention_graph_workspace_size(ctypes.byref(q), ctypes.byref(k))

    def records_bytes(batch, splits):
        records = batch * 8 * splits * 2
        return -(-records * 128 * 4 // 256) * 256 + records * 8

    assert workspace(8, 16384) == records_bytes(8, 16384 // 512)   # 8192 one-round items -> four rounds
    assert workspace(1, 4096) == records_bytes(1, 4096 // 128)     # 256 one-round items
    assert workspace(16, 16384) == records_bytes(16, 16384 // 128)  # 4096 four-round items: one round
    assert lib.xinfer_status_string(18).decode() == "Graph-capture attention takes at most 64 rows"

    def prefill_workspace(batch, tokens, capacity, hq=16, hkv=8, dim=128):
        q, k = view([batch, hq, tokens, dim]), view([batch, hkv, capacity, dim])
        return lib.xinfer_batched_flash_attention_graph_workspace_size(ctypes.byref(q), ctypes.byref(k))

    def prefill_records_bytes(units, splits, dim=128):
        records = min(2048 + units, units * splits) * 128
        return -(-records * dim * 4 // 256) * 256 + records * 8

    for (batch, tokens, capacity, splits) in [(4, 128, 4096, 8), (8, 512, 16384, 8), (2, 64, 1024, 2)]:
        units = batch * 8 * -(-tokens * 2 // 128)
        size, records = prefill_workspace(batch, tokens, capacity), prefill_records_bytes(units, splits)
        assert records < size < records + 8192, (batch, tokens, capacity)
    assert prefill_workspace(2, 64, 512) < 8192  # 512 keys: never split, no records

    def graph(qv, kv):
        return lib.xinfer_batched_flash_attention_graph(ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(kv),
                                                        ctypes.c_void_p(1 << 21), None, ctypes.c_int64(0),
                                                        ctypes.c_double(0.1), ctypes.c_void_p(1 << 20), None,
                                                        ctypes.c_size_t(0), None)

    assert graph(view([1, 16, 5, 128]), view([1, 8, 256, 128])) == 10   # prefill shapes: no workspace given
    assert graph(view([65, 16, 1, 128]), view([65, 8, 256, 128])) == 18
    assert graph(view([1, 16, 1, 128]), view([1, 8, 256, 128])) == 10   # no workspace given
    qv, kv = view([2, 16, 64, 128]), view([2, 8, 1024, 128])
    size = lib.xinfer_batched_flash_attention_graph_workspace_size(ctypes.byref(qv), ctypes.byref(kv))
    misaligned = lib.xinfer_batched_flash_attention_graph(
        ctypes.byref(qv), ctypes.byref(kv), ctypes.byref(kv), ctypes.c_void_p(1 << 21), None, ctypes.c_int64(0),
        ctypes.c_double(0.1), ctypes.c_void_p(1 << 20), ctypes.c_void_p((1 << 22) + 4), ctypes.c_size_t(size), None)
    assert misaligned == 10
    assert lib.xinfer_batched_flash_attention_graph_workspace_size(ctypes.byref(view([1, 16, 1, 128])),
                                                                   ctypes.byref(view([1, 8, 128, 128]))) == 0


def prefill_records(lib, counts, lengths, hq, hkv, d, capacity):
    """Partial records the planner lays out for a batched prefill call."""
    q, k = view([len(counts), hq, max(counts), d]), view([len(counts), hkv, capacity, d])
    offsets = [0]
    for count in counts:
        offsets.append(offsets[-1] + count)
    offsets.append(0)
    for length in lengths:
        offsets.append(offsets[-1] + length)
    host = (ctypes.c_int32 * len(offsets))(*offsets)
    bytes_ = lib.xinfer_batched_flash_attention_workspace_size(ctypes.byref(q), ctypes.byref(k), host)
    return bytes_ // (d * 4 + 8)


def test_prefill_split_choice(lib):
    """Uniform rows keep about 256 items (4 splits of each 128-vector query
    tile here); a ragged batch whose rows differ 7x in length is cut finer, so
    that no single item holds a long row's keys."""
    # cfg2: one 512-token chunk at offset 1536 -> 64 query tiles x 4 splits x 128 vectors.
    assert prefill_records(lib, [512], [2048], 16, 8, 128, 4096) == 64 * 4 * 128
    # The same chunk at offset 15872: still 4 splits (4096 keys each).
    assert prefill_records(lib, [512], [16384], 16, 8, 128, 16384) == 64 * 4 * 128
    # cfg5 (D = 256, ragged): 300 query tiles; the 9315-key row is split too.
    counts = [356, 138, 422, 459, 325, 298, 113, 124]
    lengths = [14244, 13896, 2059, 4214, 12262, 14086, 12837, 9315]
    tiles = sum(4 * -(-count * 4 // 128) for count in counts)
    assert prefill_records(lib, counts, lengths, 16, 4, 256, 16384) > 3 * tiles * 128
    # The split the dispatch model picks among every row's split-count change
    # points: 3200-key splits (5, 5, 1, 2, 4, 5, 5, 3 splits per row; 241 split
    # tiles per kv head), measured faster than the 2752-key splits of octave
    # steps and than 3264-key splits (one split fewer on the 12837-key row).
    assert prefill_records(lib, counts, lengths, 16, 4, 256, 16384) == 4 * 241 * 128


def test_plans_are_recomputed_when_the_call_changes(lib):
    """The per-thread cache of the last plan: alternating calls, each asking
    for its workspace twice, get the workspace of a fresh plan every time."""
    counts = [356, 138, 422, 459, 325, 298, 113, 124]
    lengths = [14244, 13896, 2059, 4214, 12262, 14086, 12837, 9315]
    ragged = prefill_records(lib, counts, lengths, 16, 4, 256, 16384)
    uniform = prefill_records(lib, [512], [2048], 16, 8, 128, 4096)
    for _ in range(2):
        assert prefill_records(lib, counts, lengths, 16, 4, 256, 16384) == ragged
        assert prefill_records(lib, counts, lengths, 16, 4, 256, 16384) == ragged
        assert prefill_records(lib, [512], [2048], 16, 8, 128, 4096) == uniform
        # Same counts and lengths, other geometry: its own plan.
        assert prefill_records(lib, [512], [2048], 16, 8, 64, 4096) == uniform
        assert prefill_records(lib, [512], [2048], 16, 8, 128, 4096) == uniform
        shorter = [length - 1000 for length in lengths]
        assert prefill_records(lib, counts, shorter, 16, 4, 256, 16384) != ragged


def decode_workspace(lib, counts, lengths, hq, hkv, d, capacity):
    q, k = view([len(counts), hq, max(counts), d]), view([len(counts), hkv, capacity, d])
    offsets = [0]
    for count in counts:
        offsets.append(offsets[-1] + count)
    offsets.append(0)
    for length in lengths:
        offsets.append(offsets[-1] + length)
    host = (ctypes.c_int32 * len(offsets))(*offsets)
    return lib.xinfer_batched_flash_attention_workspace_size(ctypes.byref(q), ctypes.byref(k), host)


def expected_workspace(records, d, counters):
    """capi.cpp's layout: fp32 outputs, then (m, l) pairs, then the decode
    launch's arrival counters, each region starting on a 256-byte boundary."""
    align = lambda n: -(-n // 256) * 256
    return align(align(records * d * 4) + records * 8) + counters * 8


def test_decode_item_rounds_and_in_launch_merge_counters(lib):
    """The planner's decode choices, read from the workspace it asks for.

    Head dim 128, 16 query / 8 KV heads, one query per row: 2 query vectors
    per KV head, 128 keys per one-round item, 512 per four-round item.  A
    launch whose split rows all have at most 8 splits (and Hkv a multiple of
    8) gets one arrival counter per decode item for the in-launch merge."""
    # cfg1: one row of 1024 keys, one-round items, 8 splits: in-launch merge.
    assert decode_workspace(lib, [1], [1024], 16, 8, 128, 4096) == expected_workspace(8 * 8 * 2, 128, 8 * 8)
    # cfg3 seed 1's lengths: the 2170-key row has 17 one-round splits; four
    # rounds would fit the in-launch merge, but the latency model keeps one
    # round and the merge launch.
    lengths = [24, 75, 81, 54, 755, 34, 390, 2170]
    splits = [-(-length // 128) for length in lengths]
    records = 8 * 2 * sum(s for s in splits if s > 1)
    assert decode_workspace(lib, [1] * 8, lengths, 16, 8, 128, 16384) == expected_workspace(records, 128, 0)
    # cfg3 seed 3's lengths: four-round items bring the longest row to 7
    # splits, and the model takes them with the in-launch merge.
    lengths = [20, 116, 3394, 53, 3006, 1084, 63, 322]
    splits = [-(-length // 512) for length in lengths]
    records = 8 * 2 * sum(s for s in splits if s > 1)
    assert decode_workspace(lib, [1] * 8, lengths, 16, 8, 128, 16384) == expected_workspace(
        records, 128, 8 * sum(splits))
    # Four KV heads: no in-launch merge, whatever the splits.
    assert decode_workspace(lib, [1], [1024], 16, 4, 128, 4096) == expected_workspace(4 * 8 * 4, 128, 0)
    # Nine splits: past the in-launch merge's layout.
    assert decode_workspace(lib, [1], [1100], 16, 8, 128, 4096) == expected_workspace(8 * 9 * 2, 128, 0)


def test_operator_schemas_tags_and_fakes(library_path):
    from xinfer_amd.attention import attention_c_shims, cache_extent, load_attention_ops

    load_attention_ops(library_path)
    for name, schema in REFERENCE_SCHEMAS.items():
        op = getattr(torch.ops.xinfer, name).default
        assert str(op._schema) == schema
    assert torch.Tag.flexible_layout in torch.ops.xinfer.flash_attention.default.tags
    assert torch.Tag.flexible_layout in torch.ops.xinfer.batched_flash_attention.default.tags
    shims = attention_c_shims()
    assert len(shims) == 6
    assert all(name in text[0] for name, text in zip(
        ("aoti_torch_cuda_flash_attention", "aoti_torch_cuda_batched_flash_attention",
         "aoti_torch_cuda_append_kv_batched", "aoti_torch_cuda_qk_norm_rope_append",
         "aoti_torch_cuda_batched_flash_attention_bthd", "aoti_torch_cuda_projection_gemv"), shims.values()))
    with FakeTensorMode(allow_non_fake_inputs=True):
        q = torch.empty(2, 16, 3, 128, dtype=torch.bfloat16, device="cuda").transpose(1, 2).contiguous().transpose(1, 2)
        k = torch.empty(2, 8, 64, 128, dtype=torch.bfloat16, device="cuda")
        out = torch.ops.xinfer.flash_attention(q, k, k, cache_extent(10), 0.1)
        assert out.shape == q.shape and out.is_contiguous() and out.device == q.device
        offsets = torch.zeros(2, 3, dtype=torch.int32)
        cuda_offsets = torch.empty(2, 3, dtype=torch.int32, device="cuda")
        blocks = torch.empty(2, 1, dtype=torch.int32, device="cuda")
        out = torch.ops.xinfer.batched_flash_attention(q, k, k, offsets, cuda_offsets, blocks, 0.1)
        assert out.shape == q.shape and out.is_contiguous()
        positions = torch.empty(2, 3, dtype=torch.long, device="cuda")
        cu = torch.empty(3, dtype=torch.int32, device="cuda")
        assert torch.ops.xinfer.append_kv_batched(k[:, :, :3], k[:, :, :3], positions, cu, k, k) is None
        # The fake contract rejects what the native op rejects.
        with pytest.raises(Exception):
            torch.ops.xinfer.flash_attention(q[:, :3], k, k, cache_extent(10), 0.1)
        with pytest.raises(Exception):
            torch.ops.xinfer.batched_flash_attention(q, k, k, offsets[:, :2], cuda_offsets, blocks, 0.1)
