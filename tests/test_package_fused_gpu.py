"""The fused step before the attention, and the [B, T, Hq, D] output variant, in packages.

The model-step packages (test_package_model_gpu.py) hold Inductor's own
kernels around the native operators, so they meet eager within bounds.  This
step holds nothing but native operators: per layer, ``qk_norm_rope_append``
(q/k RMSNorm, rotary embedding and the K/V append in one launch), then
``batched_flash_attention_bthd``, over per-head projections, rotary tables and
positions given as inputs and the two RMSNorm weights held as module
parameters (package constants).  It is exported with batch in [1, 8] (prefill
tokens in [2, 512]) as the reference's exporter does
(compiler/qwen3/export.py:27-56), packaged with the library, and run in a
fresh process that takes the library out of the package.  For B = 1..8 over
the reference's count patterns (compiler/qwen3/tests/test_export.py:101-155)
the package must equal the eager step bit for bit -- outputs and caches --
with every cache slot outside each row's append, and every row past the
batch, unchanged.
"""

import json
import os
from pathlib import Path
import subprocess
import sys
import textwrap

import pytest
import torch
from torch.fx.experimental import _config as symbolic_config

from xinfer_amd.adapters import MAX_BATCH_SIZE, MAX_PREFILL
from attn_helpers import log

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
LAYERS, HEADS, KV_HEADS, DIM, CAPACITY = 2, 16, 8, 128, 1024
EPS, SCALE = 1e-6, DIM**-0.5


class FusedStep(torch.nn.Module):
    """Metadata once, then per layer the fused norm/rope/append and the [B, T, Hq, D] attention."""

    def __init__(self):
        super().__init__()
        generator = torch.Generator().manual_seed(11)
        self.q_weight = torch.nn.Parameter((1 + 0.2 * torch.randn(DIM, generator=generator)).to(torch.bfloat16),
                                           requires_grad=False)
        self.k_weight = torch.nn.Parameter((1 + 0.2 * torch.randn(DIM, generator=generator)).to(torch.bfloat16),
                                           requires_grad=False)

    def forward(self, queries, keys, values, cos, sin, positions, kv, kv_lengths, query_lengths):
        from xinfer_amd.attention import batched_attention_metadata

        offsets, cuda_offsets, blocks = batched_attention_metadata(kv_lengths, query_lengths, positions.device)
        outputs = []
        for layer in range(LAYERS):
            k, v = kv[2 * layer], kv[2 * layer + 1]
            q = torch.ops.xinfer.qk_norm_rope_append(queries[layer], keys[layer], values[layer], self.q_weight,
                                                     self.k_weight, EPS, cos, sin, positions, cuda_offsets[0], k, v)
            outputs.append(torch.ops.xinfer.batched_flash_attention_bthd(q, k, v, offsets, cuda_offsets, blocks,
                                                                         SCALE))
        return tuple(outputs)


def step_inputs(batch, width, starts, counts, generator=None, device="cuda"):
    """Per-head projections, rotary tables of the positions, caches and lengths."""
    options = dict(device=device, dtype=torch.bfloat16)
    queries = tuple(torch.randn(batch, width, HEADS, DIM, generator=generator, device=device).to(torch.bfloat16)
                    for _ in range(LAYERS))
    keys = tuple(torch.randn(batch, width, KV_HEADS, DIM, generator=generator, device=device).to(torch.bfloat16)
                 for _ in range(LAYERS))
    values = tuple(torch.randn(batch, width, KV_HEADS, DIM, generator=generator, device=device).to(torch.bfloat16)
                   for _ in range(LAYERS))
    positions = torch.stack([torch.arange(s, s + width, device=device) for s in starts])
    inv_freq = 1.0 / (1e6 ** (torch.arange(0, DIM, 2, device=device, dtype=torch.float32) / DIM))
    angles = positions[..., None].float() * inv_freq
    angles = torch.cat((angles, angles), dim=-1)
    cos, sin = angles.cos().to(torch.bfloat16), angles.sin().to(torch.bfloat16)
    kv = tuple(torch.zeros(batch, KV_HEADS, CAPACITY, DIM, **options) for _ in range(2 * LAYERS))
    lengths = torch.tensor([s + c for s, c in zip(starts, counts)], dtype=torch.int32)
    return queries, keys, values, cos, sin, positions, kv, lengths, torch.tensor(counts, dtype=torch.int32)


def export_step(step, kind):
    batch_size, width = 2, (1 if kind == "decode" else 16)
    starts = [16 + 8 * row for row in range(batch_size)]
    counts = [max(1, width // (row + 1)) for row in range(batch_size)]
    inputs = step_inputs(batch_size, width, starts, counts)
    batch = torch.export.Dim("batch", min=1, max=MAX_BATCH_SIZE)
    token_shape = {0: batch}
    if kind == "prefill":
        token_shape[1] = torch.export.Dim("tokens", min=2, max=MAX_PREFILL)
    per_layer = tuple(token_shape for _ in range(LAYERS))
    shapes = (per_layer, per_layer, per_layer, token_shape, token_shape, token_shape,
              tuple({0: batch} for _ in range(2 * LAYERS)), {0: batch}, {0: batch})
    with symbolic_config.patch(backed_size_oblivious=True):
        exported = torch.export.export(step, inputs, dynamic_shapes=shapes, strict=False)
    exported.validate()
    return exported


@pytest.fixture(scope="module")
def bundle(gpu_ops, tmp_path_factory):
    from xinfer_amd.attention import attention_c_shims, attention_library
    from xinfer_amd.package import compile_package

    directory = tmp_path_factory.mktemp("fused")
    step = FusedStep().cuda()
    programs = {}
    for kind in ("prefill", "decode"):
        log(f"export + AOTI package of the fused {kind} step")
        with torch.inference_mode():
            program = export_step(step, kind)
            compile_package(program, directory / f"{kind}.pt2", inductor_configs={"emulate_precision_casts": True},
                            native_libraries=[Path(attention_library())], custom_op_shims=attention_c_shims())
        programs[kind] = program
    return directory, programs


def test_fused_graphs_hold_only_the_native_steps(bundle, gpu_ops):
    _, programs = bundle
    for kind, program in programs.items():
        targets = [node.target for node in program.graph.nodes if node.op == "call_function"]
        assert targets.count(gpu_ops.qk_norm_rope_append.default) == LAYERS
        assert targets.count(gpu_ops.batched_flash_attention_bthd.default) == LAYERS
        assert gpu_ops.append_kv_batched.default not in targets
        assert gpu_ops.batched_flash_attention.default not in targets
        assert torch.ops.aten.index_copy.default not in targets
        assert not program.graph_signature.buffers_to_mutate


WORKER = textwrap.dedent(
    """
    import json, sys
    from pathlib import Path
    sys.path.insert(0, sys.argv[1])
    sys.path.insert(0, sys.argv[1] + '/tests')
    import torch
    from xinfer_amd.validation import load_packaged_attention_ops
    from xinfer_amd.package import load_package
    from test_package_fused_gpu import FusedStep, step_inputs, LAYERS

    directory = Path(sys.argv[2])
    extracted = load_packaged_attention_ops(directory)
    step = FusedStep().cuda()
    PATTERNS = {'decode': ((1,), (0, 1), (1, 0)), 'prefill': ((7, 16), (1, 2), (0, 16), (512, 1))}

    def bits_equal(a, b):
        return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))

    checks = 0
    with torch.inference_mode():
        for kind in ('prefill', 'decode'):
            package = load_package(directory / f'{kind}.pt2')
            for batch in range(1, 9):
                for pattern in PATTERNS[kind]:
                    counts = [pattern[row % len(pattern)] for row in range(batch)]
                    if not max(counts):
                        continue
                    case = f'{kind} batch={batch} counts={counts}'
                    print(case, file=sys.stderr, flush=True)
                    width = max(max(counts), 2 if kind == 'prefill' else 1)
                    starts = [0 if count == 512 else 3 + row for row, count in enumerate(counts)]
                    generator = torch.Generator(device='cuda').manual_seed(1000 * batch + checks)
                    queries, keys, values, cos, sin, positions, _, lengths, query_lengths = step_inputs(
                        batch, width, starts, counts, generator)
                    initial = tuple(torch.randn(8, 8, 1024, 128, generator=generator, device='cuda').to(torch.bfloat16)
                                    for _ in range(2 * LAYERS))
                    results = []
                    for call in (step, package):
                        state = tuple(t.clone() for t in initial)
                        out = call(queries, keys, values, cos, sin, positions, tuple(t[:batch] for t in state),
                                   lengths, query_lengths)
                        results.append((out, state))
                    torch.cuda.synchronize()
                    (eager, eager_state), (packaged, package_state) = results
                    if not all(bits_equal(a, b) for a, b in zip(eager, packaged)):
                        raise AssertionError(f'package output differs from eager: {case}')
                    if not all(bits_equal(a, b) for a, b in zip(eager_state, package_state)):
                        raise AssertionError(f'package caches differ from eager: {case}')
                    for before, after in zip(initial, package_state):
                        if not bits_equal(before[batch:], after[batch:]):
                            raise AssertionError(f'rows past the batch changed: {case}')
                        for row, (start, count) in enumerate(zip(starts, counts)):
                            if not (bits_equal(before[row, :, :start], after[row, :, :start])
                                    and bits_equal(before[row, :, start + count:], after[row, :, start + count:])):
                                raise AssertionError(f'cache slot outside the append changed: {case}')
                    for out in packaged:
                        if not bool(torch.isfinite(out).all()):
                            raise AssertionError(f'nonfinite output: {case}')
                    checks += 1
    paths = {line.split(maxsplit=5)[5].removesuffix(' (deleted)')
             for line in Path('/proc/self/maps').read_text().splitlines() if 'libxinfer_attention_ops.so' in line}
    if paths != {str(extracted)}:
        raise AssertionError(f'not the packaged library: {paths}')
    print(json.dumps(dict(checks=checks)), flush=True)
    """
)


def test_fused_packages_equal_eager_in_a_fresh_process(bundle):
    directory, _ = bundle
    env = dict(os.environ, XINFER_ATTENTION_OPS_LIBRARY="/nonexistent/attention.so")
    env.pop("PYTHONPATH", None)
    log("fresh process, fused-step packages")
    result = subprocess.run([sys.executable, "-c", WORKER, str(ROOT), str(directory)], env=env,
                            capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stdout[-4000:] + result.stderr[-4000:]
    report = json.loads(result.stdout.splitlines()[-1])
    assert report["checks"] == (3 * 8 - 1) + (4 * 8 - 1)
