"""The batched operators inside AOTInductor packages with dynamic batch and tokens.

Counterpart of the reference's export and package checks of the batched path:
compiler/qwen3/export.py:27-56 exports each entry point with batch in [1, 8]
(and prefill tokens in [2, 512]) under backed_size_oblivious, and
compiler/qwen3/tests/test_export.py:86-169 requires one batched_flash_attention
and one append_kv_batched node per layer, no mutated buffers, B = 1..8 equal
to eager bit for bit over ragged count patterns (inactive rows included),
untouched cache slots unchanged, and errors from the exported module for
B = 0 and B = 9.

The exported module is the attention part of ModelStep.forward: the step's
metadata is built once from the CPU lengths (KVCache.__init__,
compiler/qwen3/model.py:37-47), then every layer appends its new K/V and runs
the batched attention on the adapters' transposed [B, T, H, D] views
(compiler/qwen3/adapters/attention.py:49-60).  prefill.pt2 and decode.pt2 are
built with the library and its C shims; fresh processes that never load the
library themselves load them in both orders, and a third process first takes
the library out of prefill.pt2 for eager validation
(tools/validation/common/attention.py:29-51) and then loads the packages.
"""

import json
import os
from pathlib import Path
import subprocess
import sys
import textwrap
import zipfile

import pytest
import torch
from torch.fx.experimental import _config as symbolic_config

from xinfer_amd.adapters import MAX_BATCH_SIZE, MAX_PREFILL
from attn_helpers import log
from xinfer_amd.attention import batched_attention_metadata

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
LAYERS, HEADS, KV_HEADS, DIM, CAPACITY = 2, 16, 8, 128, 1024
SCALE = DIM**-0.5


class BatchedStep(torch.nn.Module):
    """Metadata once, then per layer: the append, then the batched attention."""

    def forward(self, queries, keys, values, positions, kv, kv_lengths, query_lengths):
        offsets, cuda_offsets, blocks = batched_attention_metadata(kv_lengths, query_lengths, positions.device)
        outputs = []
        for layer in range(LAYERS):
            k, v = kv[2 * layer], kv[2 * layer + 1]
            torch.ops.xinfer.append_kv_batched(keys[layer].transpose(1, 2), values[layer].transpose(1, 2),
                                               positions, cuda_offsets[0], k, v)
            outputs.append(torch.ops.xinfer.batched_flash_attention(
                queries[layer].transpose(1, 2), k, v, offsets, cuda_offsets, blocks, SCALE))
        return tuple(outputs)


def example_inputs(kind):
    """Tracing inputs shaped like the reference exporter's (batch 2, starts 16 + 8 row)."""
    batch, width = 2, (1 if kind == "decode" else 16)
    starts = [16 + 8 * row for row in range(batch)]
    counts = [max(1, width // (row + 1)) for row in range(batch)]
    options = dict(device="cuda", dtype=torch.bfloat16)
    queries = tuple(torch.randn(batch, width, HEADS, DIM, **options) for _ in range(LAYERS))
    keys = tuple(torch.randn(batch, width, KV_HEADS, DIM, **options) for _ in range(LAYERS))
    values = tuple(torch.randn(batch, width, KV_HEADS, DIM, **options) for _ in range(LAYERS))
    positions = torch.stack([torch.arange(s, s + width, device="cuda") for s in starts])
    kv = tuple(torch.zeros(batch, KV_HEADS, CAPACITY, DIM, **options) for _ in range(2 * LAYERS))
    lengths = torch.tensor([s + c for s, c in zip(starts, counts)], dtype=torch.int32)
    return queries, keys, values, positions, kv, lengths, torch.tensor(counts, dtype=torch.int32)


def export_step(kind):
    batch = torch.export.Dim("batch", min=1, max=MAX_BATCH_SIZE)
    token_shape = {0: batch}
    if kind == "prefill":
        token_shape[1] = torch.export.Dim("tokens", min=2, max=MAX_PREFILL)
    per_layer = tuple(token_shape for _ in range(LAYERS))
    shapes = (per_layer, per_layer, per_layer, token_shape, tuple({0: batch} for _ in range(2 * LAYERS)),
              {0: batch}, {0: batch})
    with symbolic_config.patch(backed_size_oblivious=True):
        exported = torch.export.export(BatchedStep(), example_inputs(kind), dynamic_shapes=shapes, strict=False)
    exported.validate()
    return exported


@pytest.fixture(scope="module")
def bundle(gpu_ops, tmp_path_factory):
    from xinfer_amd.attention import attention_c_shims, attention_library
    from xinfer_amd.package import compile_package

    library = Path(attention_library())
    directory = tmp_path_factory.mktemp("bundle")
    programs = {}
    for kind in ("prefill", "decode"):
        log(f"export + AOTI package of the batched {kind} step")
        with torch.inference_mode():
            program = export_step(kind)
            compile_package(program, directory / f"{kind}.pt2", inductor_configs={}, native_libraries=[library],
                            custom_op_shims=attention_c_shims())
        programs[kind] = program
    return directory, library, programs


def test_exported_graphs_hold_the_native_ops_with_dynamic_batch(bundle, gpu_ops):
    _, _, programs = bundle
    for kind, program in programs.items():
        log(f"exported graph {kind}")
        placeholders = [node for node in program.graph.nodes if node.op == "placeholder"]
        positions = next(node for node in placeholders if node.target == "positions")
        batch = positions.meta["val"].shape[0]
        constraint = program.range_constraints[batch.node.expr]
        assert (constraint.lower, constraint.upper) == (1, 8)
        if kind == "prefill":
            tokens = positions.meta["val"].shape[1]
            constraint = program.range_constraints[tokens.node.expr]
            assert (constraint.lower, constraint.upper) == (2, 512)
        assert not program.graph_signature.buffers_to_mutate
        targets = [node.target for node in program.graph.nodes if node.op == "call_function"]
        assert targets.count(gpu_ops.batched_flash_attention.default) == LAYERS
        assert targets.count(gpu_ops.append_kv_batched.default) == LAYERS
        assert torch.ops.aten.index_copy.default not in targets
        assert torch.ops.aten.scaled_dot_product_attention.default not in targets
        # The exported module's range guard rejects B = 9
        # (compiler/qwen3/tests/test_export.py:156-169).  This PyTorch's guards
        # do not enforce the lower bound, so B = 0 may also run: it must then
        # return empty outputs.
        width = 1 if kind == "decode" else 2
        options = dict(device="cuda", dtype=torch.bfloat16)
        for batch in (0, 9):
            bad = (tuple(torch.zeros(batch, width, HEADS, DIM, **options) for _ in range(LAYERS)),
                   tuple(torch.zeros(batch, width, KV_HEADS, DIM, **options) for _ in range(LAYERS)),
                   tuple(torch.zeros(batch, width, KV_HEADS, DIM, **options) for _ in range(LAYERS)),
                   torch.zeros(batch, width, dtype=torch.int64, device="cuda"),
                   tuple(torch.zeros(batch, KV_HEADS, CAPACITY, DIM, **options) for _ in range(2 * LAYERS)),
                   torch.ones(batch, dtype=torch.int32), torch.ones(batch, dtype=torch.int32))
            try:
                with torch.inference_mode():
                    outputs = program.module()(*bad)
            except (RuntimeError, AssertionError):
                continue
            assert batch == 0, f"batch {batch} accepted by the exported {kind} module"
            assert all(out.shape == (0, HEADS, width, DIM) for out in outputs)


def test_packages_call_the_batched_shims(bundle):
    directory, library, _ = bundle
    for kind in ("prefill", "decode"):
        with zipfile.ZipFile(directory / f"{kind}.pt2") as archive:
            names = archive.namelist()
            carried = [name for name in names if "/data/aotinductor/" in name and name.endswith("/" + library.name)]
            assert len(carried) == 1 and archive.read(carried[0]) == library.read_bytes()
            sources = b"\n".join(archive.read(name) for name in names if name.endswith(".wrapper.cpp")).decode()
        attention = "AOTI_TORCH_ERROR_CODE_CHECK(aoti_torch_cuda_batched_flash_attention("
        append = "AOTI_TORCH_ERROR_CODE_CHECK(aoti_torch_cuda_append_kv_batched("
        assert sources.count(attention) == LAYERS and sources.count(append) == LAYERS
        assert sources.index("AOTICudaStreamGuard") < sources.index(append) < sources.index(attention)
        assert "aoti_torch_proxy_executor_call_function" not in sources


WORKER = textwrap.dedent(
    """
    import gc, json, sys
    from pathlib import Path
    sys.path.insert(0, sys.argv[1])
    import torch
    from xinfer_amd.attention import batched_attention_metadata
    from xinfer_amd.package import load_package

    directory, build_library, mode = Path(sys.argv[2]), Path(sys.argv[3]), sys.argv[4]
    LAYERS, HEADS, KV_HEADS, DIM, CAPACITY = 2, 16, 8, 128, 1024
    SCALE = DIM ** -0.5
    MAX_ABS, MEAN_ABS = 2e-2, 2e-3
    PATTERNS = {'decode': ((1,), (0, 1), (1, 0)), 'prefill': ((7, 16), (1, 2), (0, 16), (512, 1))}

    if mode == 'validation':
        from xinfer_amd.validation import load_packaged_attention_ops
        extracted = load_packaged_attention_ops(directory)
        order = ['prefill', 'decode']
    else:
        extracted = None
        order = mode.split(',')

    def eager_step(queries, keys, values, positions, kv, kv_lengths, query_lengths):
        offsets, cuda_offsets, blocks = batched_attention_metadata(kv_lengths, query_lengths, positions.device)
        outputs = []
        for layer in range(LAYERS):
            k, v = kv[2 * layer], kv[2 * layer + 1]
            torch.ops.xinfer.append_kv_batched(keys[layer].transpose(1, 2), values[layer].transpose(1, 2),
                                               positions, cuda_offsets[0], k, v)
            outputs.append(torch.ops.xinfer.batched_flash_attention(
                queries[layer].transpose(1, 2), k, v, offsets, cuda_offsets, blocks, SCALE))
        return tuple(outputs)

    def fp32_reference(q, k, v, counts, lengths):
        out = torch.zeros(q.shape, dtype=torch.float32, device='cuda')
        for r, (count, length) in enumerate(zip(counts, lengths)):
            if not count:
                continue
            qr = q[r, :, :count].float().contiguous()
            kr = k[r, :, :length].float().repeat_interleave(HEADS // KV_HEADS, 0)
            vr = v[r, :, :length].float().repeat_interleave(HEADS // KV_HEADS, 0).contiguous()
            s = torch.matmul(qr, kr.transpose(1, 2).contiguous()) * SCALE
            hidden = torch.arange(length, device='cuda')[None, :] > (length - count + torch.arange(count, device='cuda'))[:, None]
            out[r, :, :count] = torch.matmul(s.masked_fill(hidden, float('-inf')).softmax(-1), vr)
        return out

    def bits_equal(a, b):
        return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))

    checks = []
    models = {kind: load_package(directory / f'{kind}.pt2') for kind in order}
    for kind, model in models.items():
        for batch in range(1, 9):
            for pattern in PATTERNS[kind]:
                counts = [pattern[row % len(pattern)] for row in range(batch)]
                if not max(counts):
                    continue
                torch.manual_seed(1000 * batch + len(checks))
                width = max(max(counts), 2 if kind == 'prefill' else 1)
                starts = [0 if count == 512 else 3 + row for row, count in enumerate(counts)]
                options = dict(device='cuda', dtype=torch.bfloat16)
                queries = tuple(torch.randn(batch, width, HEADS, DIM, **options) for _ in range(LAYERS))
                keys = tuple(torch.randn(batch, width, KV_HEADS, DIM, **options) for _ in range(LAYERS))
                values = tuple(torch.randn(batch, width, KV_HEADS, DIM, **options) for _ in range(LAYERS))
                positions = torch.stack([torch.arange(s, s + width, device='cuda') for s in starts])
                initial = tuple(torch.randn(8, KV_HEADS, CAPACITY, DIM, **options) for _ in range(2 * LAYERS))
                lengths = torch.tensor([s + c for s, c in zip(starts, counts)], dtype=torch.int32)
                query_lengths = torch.tensor(counts, dtype=torch.int32)
                results = []
                with torch.inference_mode():
                    for call in (eager_step, model):
                        state = tuple(t.clone() for t in initial)
                        outputs = call(queries, keys, values, positions, tuple(t[:batch] for t in state),
                                       lengths, query_lengths)
                        results.append((outputs, state))
                torch.cuda.synchronize()
                (eager_out, eager_state), (pkg_out, pkg_state) = results
                case = f'{kind} batch={batch} counts={counts}'
                if not all(bits_equal(a, b) for a, b in zip(eager_out, pkg_out)):
                    raise AssertionError(f'package output differs from eager: {case}')
                if not all(bits_equal(a, b) for a, b in zip(eager_state, pkg_state)):
                    raise AssertionError(f'package cache differs from eager: {case}')
                for before, after in zip(initial, pkg_state):
                    if not bits_equal(before[batch:], after[batch:]):
                        raise AssertionError(f'rows past the batch changed: {case}')
                    for row, (start, count) in enumerate(zip(starts, counts)):
                        if not (bits_equal(before[row, :, :start], after[row, :, :start])
                                and bits_equal(before[row, :, start + count:], after[row, :, start + count:])):
                            raise AssertionError(f'cache slot outside the append changed: {case}')
                layer = len(checks) % LAYERS
                k, v = pkg_state[2 * layer], pkg_state[2 * layer + 1]
                expected = fp32_reference(queries[layer].transpose(1, 2), k, v, counts, lengths.tolist())
                out = pkg_out[layer]
                for row, count in enumerate(counts):
                    if torch.count_nonzero(out[row, :, count:]).item():
                        raise AssertionError(f'padded queries not zero: {case}')
                    if count:
                        err = (out[row, :, :count].float() - expected[row, :, :count]).abs()
                        if float(err.max()) > MAX_ABS or float(err.mean()) > MEAN_ABS:
                            raise AssertionError(f'outside the fp32 gates: {case}')
                checks.append([kind, batch, counts])
    paths = {line.split(maxsplit=5)[5].removesuffix(' (deleted)')
             for line in Path('/proc/self/maps').read_text().splitlines() if 'libxinfer_attention_ops.so' in line}
    if len(paths) != 1:
        raise AssertionError(f'expected one mapped attention library: {paths}')
    library = paths.pop()
    if Path(library) == build_library:
        raise AssertionError('the build tree library was loaded')
    if extracted is not None and Path(library) != Path(extracted):
        raise AssertionError(f'packages did not reuse the extracted library: {library} vs {extracted}')
    if extracted is None and 'aotinductor' not in library:
        raise AssertionError(f'attention library not taken from the package: {library}')
    print(json.dumps(dict(mode=mode, order=order, checks=len(checks), library=library)), flush=True)
    """
)


@pytest.mark.parametrize("mode", ["prefill,decode", "decode,prefill", "validation"])
def test_fresh_processes_run_the_batched_packages(bundle, mode):
    directory, library, _ = bundle
    env = dict(os.environ, XINFER_ATTENTION_OPS_LIBRARY="/nonexistent/attention.so")
    env.pop("PYTHONPATH", None)
    log(f"fresh process, batched packages, {mode}")
    result = subprocess.run([sys.executable, "-c", WORKER, str(ROOT), str(directory), str(library), mode],
                            env=env, capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stdout[-4000:] + result.stderr[-4000:]
    report = json.loads(result.stdout.splitlines()[-1])
    # Every pattern at every batch, less the all-inactive batch of one row
    # ((0, 1) for decode, (0, 16) for prefill): 3 * 8 - 1 and 4 * 8 - 1 cases.
    assert report["checks"] == (3 * 8 - 1) + (4 * 8 - 1)
