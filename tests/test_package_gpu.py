"""The operators inside AOTInductor packages, loaded the way prefill.pt2 and
decode.pt2 are.

Counterpart of compiler/common/tests/test_package.py:186-315 (BundledAttention):
packages built from exported modules with the library and its C shims, then

* linkage: the wrapper calls the C shims directly (no proxy executor) after
  selecting the caller's stream, needs libxinfer_attention_ops.so with a
  $ORIGIN run path, and the package carries the library byte for byte;
* fresh processes that never load the library themselves load the packages in
  both orders, twice: the library comes from the package, outputs equal the
  eager operators bit for bit and the fp32 reference within the gates, inputs
  stay unchanged, the native append mutates only the caches, and a native
  error surfaces as a RuntimeError with the native message on stderr.

The reference compares against ATen's own flash kernel bit for bit; here the
eager operator is the bitwise reference and the fp32 oracle the numeric one.
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

from attn_helpers import log

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
KINDS = ("prefill", "decode", "append", "append_decode", "invalid_scale")

WORKER = textwrap.dedent(
    """
    import gc, json, sys
    from pathlib import Path
    sys.path.insert(0, sys.argv[1])
    import torch
    from xinfer_amd.package import load_package

    directory, build_library, order = Path(sys.argv[2]), Path(sys.argv[3]), sys.argv[4].split(',')
    MAX_ABS, MEAN_ABS = 2e-2, 2e-3

    def inputs(tokens, prefix):
        torch.manual_seed(23 + tokens + prefix)
        options = dict(device='cuda', dtype=torch.bfloat16)
        return (torch.randn(1, 16, tokens, 128, **options), torch.randn(1, 8, 1024, 128, **options),
                torch.randn(1, 8, 1024, 128, **options), torch.empty(prefix + 1, dtype=torch.uint8))

    def bits_equal(a, b):
        return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))

    def fp32_reference(q, k, v, prefix):
        t = q.shape[2]
        kr = k[:, :, :prefix].float().repeat_interleave(2, 1)
        vr = v[:, :, :prefix].float().repeat_interleave(2, 1)
        s = torch.matmul(q.float(), kr.transpose(2, 3).contiguous()) * 128**-0.5
        hidden = torch.arange(prefix, device='cuda')[None, :] > (prefix - t + torch.arange(t, device='cuda'))[:, None]
        return torch.matmul(s.masked_fill(hidden, float('-inf')).softmax(-1), vr.contiguous())

    def close(actual, expected):
        err = (actual.float() - expected).abs()
        return float(err.max()) <= MAX_ABS and float(err.mean()) <= MEAN_ABS

    checks, library = [], None
    for cycle in range(2):
        models = {kind: load_package(directory / f'{kind}.pt2') for kind in order}
        for kind, model in models.items():
            for prefix, prefill_tokens in ((32, 2), (512, 512), (1024, 16)):
                tokens = 1 if kind == 'decode' else prefill_tokens
                q, k, v, extent = inputs(tokens, prefix)
                saved = [t.clone() for t in (q, k, v, extent)]
                with torch.inference_mode():
                    output = model(q, k, v, extent)
                    eager = torch.ops.xinfer.flash_attention(q, k, v, extent, 128**-0.5)
                if not bits_equal(output, eager):
                    raise AssertionError(f'package differs from the eager operator: {cycle}/{kind}/{prefix}')
                if not close(output, fp32_reference(q, k, v, prefix)):
                    raise AssertionError(f'package outside the fp32 gates: {cycle}/{kind}/{prefix}')
                if not all(bits_equal(a, b) for a, b in zip((q, k, v, extent), saved)):
                    raise AssertionError('read-only attention input changed')
                if output.untyped_storage().data_ptr() in {t.untyped_storage().data_ptr() for t in (q, k, v)}:
                    raise AssertionError('attention output aliases an input')
                checks.append([cycle, kind, prefix])
        paths = {line.split(maxsplit=5)[5].removesuffix(' (deleted)')
                 for line in Path('/proc/self/maps').read_text().splitlines()
                 if 'libxinfer_attention_ops.so' in line}
        if len(paths) != 1:
            raise AssertionError(f'expected one mapped attention library: {paths}')
        library = paths.pop()
        if Path(library) == build_library or 'aotinductor' not in library:
            raise AssertionError(f'attention library not taken from the package: {library}')
        del models, model
        gc.collect()

    append = {kind: load_package(directory / f'{kind}.pt2') for kind in ('append', 'append_decode')}
    mutation_checks = 0
    for tokens, position in ((2, 0), (16, 17), (1, 511)):
        q, k, v, extent = inputs(tokens, position + tokens)
        new_k, new_v = k[:, :, :tokens].clone().mul_(2), v[:, :, :tokens].clone().mul_(3)
        positions = torch.arange(position, position + tokens, device='cuda')[None, :]
        cu_query = torch.tensor([0, tokens], dtype=torch.int32, device='cuda')
        readonly = (q, new_k, new_v, positions, cu_query, extent)
        saved = [t.clone() for t in readonly]
        expected_k, expected_v = k.clone(), v.clone()
        expected_k[:, :, position:position + tokens] = new_k
        expected_v[:, :, position:position + tokens] = new_v
        pointers = (k.data_ptr(), v.data_ptr())
        with torch.inference_mode():
            output = append['append_decode' if tokens == 1 else 'append'](q, k, v, new_k, new_v, positions, cu_query, extent)
            if isinstance(output, (tuple, list)):
                output = output[0]
            expected = torch.ops.xinfer.flash_attention(q, expected_k, expected_v, extent, 128**-0.5)
        if (k.data_ptr(), v.data_ptr()) != pointers:
            raise AssertionError('cache pointers changed')
        if not all(bits_equal(a, b) for a, b in zip(readonly, saved)):
            raise AssertionError('read-only append input changed')
        if not (bits_equal(k, expected_k) and bits_equal(v, expected_v)):
            raise AssertionError('cache differs from the expected append, untouched positions included')
        if not bits_equal(output, expected):
            raise AssertionError('attention after the append differs from the eager operator')
        mutation_checks += 1

    invalid = load_package(directory / 'invalid_scale.pt2')
    try:
        with torch.inference_mode():
            invalid(*inputs(1, 32))
    except RuntimeError:
        pass
    else:
        raise AssertionError('native error did not propagate')
    print(json.dumps(dict(order=order, checks=checks, library=library,
                          mutation_checks=mutation_checks, native_error_propagated=True)), flush=True)
    """
)


class Attention(torch.nn.Module):
    def __init__(self, scale=128**-0.5):
        super().__init__()
        self.scale = scale

    def forward(self, q, k, v, extent):
        return torch.ops.xinfer.flash_attention(q, k, v, extent, self.scale)


class AppendAttention(Attention):
    """The adapters' order: the native append, then attention over the caches."""

    def forward(self, q, k, v, new_k, new_v, positions, cu_query, extent):
        torch.ops.xinfer.append_kv_batched(new_k, new_v, positions, cu_query, k, v)
        return super().forward(q, k, v, extent)


@pytest.fixture(scope="module")
def packages(gpu_ops, tmp_path_factory):
    from xinfer_amd.attention import attention_c_shims, attention_library
    from xinfer_amd.package import compile_package

    library = Path(attention_library())
    directory = tmp_path_factory.mktemp("packages")
    options = dict(device="cuda", dtype=torch.bfloat16)
    for kind in KINDS:
        tokens = 16 if kind in ("prefill", "append") else 1
        log(f"AOTI package {kind} (tokens {tokens})")
        q = torch.randn(1, 16, tokens, 128, **options)
        k = torch.randn(1, 8, 1024, 128, **options)
        v = torch.randn(1, 8, 1024, 128, **options)
        extent = torch.empty(33, dtype=torch.uint8)
        token_dim = {2: torch.export.Dim("tokens", min=2, max=512)} if tokens > 1 else {}
        extent_dim = {0: torch.export.Dim("extent", min=2, max=1025)}
        if kind.startswith("append"):
            positions = torch.arange(32 - tokens, 32, device="cuda")[None, :]
            cu_query = torch.tensor([0, tokens], dtype=torch.int32, device="cuda")
            module = AppendAttention()
            inputs = (q, k, v, k[:, :, :tokens].clone(), v[:, :, :tokens].clone(), positions, cu_query, extent)
            positions_dim = {1: token_dim[2]} if tokens > 1 else {}
            dynamic = (token_dim, {}, {}, token_dim, token_dim, positions_dim, {}, extent_dim)
        else:
            module = Attention(-1.0 if kind == "invalid_scale" else 128**-0.5)
            inputs = (q, k, v, extent)
            dynamic = (token_dim, {}, {}, extent_dim)
        with torch.inference_mode():
            exported = torch.export.export(module, inputs, dynamic_shapes=dynamic)
            compile_package(exported, directory / f"{kind}.pt2", inductor_configs={}, native_libraries=[library],
                            custom_op_shims=attention_c_shims())
    return directory, library


def test_packages_call_the_shims_and_carry_the_library(packages):
    directory, library = packages
    for kind in KINDS:
        log(f"package linkage {kind}")
        with zipfile.ZipFile(directory / f"{kind}.pt2") as archive:
            names = archive.namelist()
            carried = [name for name in names if name.endswith("/" + library.name)]
            assert len(carried) == 1
            assert archive.read(carried[0]) == library.read_bytes()
            sources = b"\n".join(archive.read(name) for name in names if name.endswith(".wrapper.cpp")).decode()
            call = "AOTI_TORCH_ERROR_CODE_CHECK(aoti_torch_cuda_flash_attention("
            assert call in sources
            if kind.startswith("append"):
                append = "AOTI_TORCH_ERROR_CODE_CHECK(aoti_torch_cuda_append_kv_batched("
                assert sources.index("AOTICudaStreamGuard") < sources.index(append) < sources.index(call)
            assert "aoti_torch_proxy_executor_call_function" not in sources
            assert sources.index("AOTICudaStreamGuard") < sources.index(call)
            wrappers = [name for name in names if name.endswith(".wrapper.so")]
            assert len(wrappers) == 1
            wrapper = directory / f"{kind}.wrapper.so"
            wrapper.write_bytes(archive.read(wrappers[0]))
        dynamic = subprocess.check_output(["readelf", "-d", str(wrapper)], text=True)
        assert f"Shared library: [{library.name}]" in dynamic
        assert "$ORIGIN" in [line for line in dynamic.splitlines() if "RUNPATH" in line or "RPATH" in line][0]


def test_fresh_processes_load_both_orders_from_the_packages(packages):
    directory, library = packages
    env = dict(os.environ, XINFER_ATTENTION_OPS_LIBRARY="/nonexistent/attention.so")
    env.pop("PYTHONPATH", None)
    for order in (("prefill", "decode"), ("decode", "prefill")):
        log(f"fresh process loading {order}")
        result = subprocess.run(
            [sys.executable, "-c", WORKER, str(ROOT), str(directory), str(library), ",".join(order)],
            env=env, capture_output=True, text=True, timeout=600,
        )
        assert result.returncode == 0, result.stdout[-4000:] + result.stderr[-4000:]
        report = json.loads(result.stdout.splitlines()[-1])
        assert report["order"] == list(order)
        assert len(report["checks"]) == 12
        assert report["mutation_checks"] == 3
        assert report["native_error_propagated"]
        # This PyTorch's AOTInductor runner raises a generic "API call failed"
        # RuntimeError and writes the shim's exception text to stderr.
        assert "Attention scale must be finite and positive" in result.stderr
