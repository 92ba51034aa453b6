"""The native projection GEMV inside an AOTInductor package.

Counterpart of the packaging case of
compiler/common/tests/test_projection_gemv_cuda.py:108-128: the exported
projection is compiled into a `.pt2` whose wrapper calls the operator's C
shim (no proxy executor, no embedded Triton kernel), carries the library,
and reproduces the eager operator bit for bit in bf16 and within the
reference's fp32 limit.
"""

from pathlib import Path
import zipfile

import pytest
import torch

from attn_helpers import log, row_errors

pytestmark = pytest.mark.gpu


class Projection(torch.nn.Module):
    def forward(self, x, weight):
        return torch.ops.xinfer.projection_gemv(x, weight)


@torch.inference_mode()
def test_projection_gemv_package(gpu_ops, tmp_path):
    from xinfer_amd.attention import attention_c_shims, attention_library
    from xinfer_amd.package import compile_package, load_package

    library = Path(attention_library())
    generator = torch.Generator().manual_seed(35)
    for dtype in (torch.bfloat16, torch.float32):
        log(f"AOTI package projection_gemv {dtype}")
        x = torch.randn(1, 33, generator=generator).to(dtype).cuda()
        weight = (torch.randn(7, 33, generator=generator) / 33**0.5).to(dtype).cuda()
        exported = torch.export.export(Projection(), (x, weight), strict=True)
        path = tmp_path / f"projection-{str(dtype).split('.')[-1]}.pt2"
        compile_package(exported, path, inductor_configs={}, native_libraries=[library],
                        custom_op_shims=attention_c_shims())
        with zipfile.ZipFile(path) as archive:
            names = archive.namelist()
            sources = b"\n".join(archive.read(n) for n in names if n.endswith(".wrapper.cpp")).decode()
            assert "aoti_torch_cuda_projection_gemv(" in sources
            assert "aoti_torch_proxy_executor_call_function" not in sources
            assert sum(n.endswith("/" + library.name) for n in names) == 1
        model = load_package(path)
        actual = model(x, weight)
        eager = torch.ops.xinfer.projection_gemv(x, weight)
        expected = torch.mm(x.double().cpu(), weight.double().cpu().t()).float()
        if dtype == torch.bfloat16:
            assert torch.equal(actual, eager)
        error = row_errors(actual.float().cpu(), expected)
        assert max(error["relative_l2"], error["peak_relative"]) <= (0.01 if dtype == torch.bfloat16 else 1e-4), error
        del model
