"""GPU checks of xinfer::projection_gemv, mirroring the reference's op tests.

Counterpart of compiler/common/tests/test_projection_gemv_cuda.py:1-130: the
profiled decoder geometries against an independent float64 CPU product (the
reference's control), exact binary inputs whose bf16 result must be bitwise
the rounded exact sum, masked tails (k not a multiple of the 16-byte step),
offset and zero-stride singleton layouts on a non-default stream, repeats,
read-only inputs, fresh output storage and the reference's error messages.
The reference's limits: bf16 relative L2 and peak relative error <= 0.01,
fp32 <= 1e-4.  (The AOTI packaging case is covered for this library's
operators by tests/test_package_gpu.py.)
"""

import pytest
import torch

from attn_helpers import log, row_errors

pytestmark = pytest.mark.gpu

DTYPES = (torch.bfloat16, torch.float32)
LIMITS = {torch.bfloat16: 0.01, torch.float32: 1e-4}
ABS_LIMITS = {torch.bfloat16: 0.0, torch.float32: 1e-7}
SHAPES = ((8224, 1024), (1024, 2048), (7168, 1024), (1024, 3584), (5120, 1024))


def inputs(n, k, dtype, *, binary=False, rank=2, zero_stride=False):
    generator = torch.Generator().manual_seed(35)
    x = torch.randn(1, k, generator=generator).to(dtype)
    weight = (torch.randn(n, k, generator=generator) / k**0.5).to(dtype)
    if binary:
        x = ((torch.arange(k) % 11 - 5) / 16).to(dtype).view(1, k)
        weight = ((torch.arange(n * k).view(n, k) % 9 - 4) / 16).to(dtype)
    expected = torch.mm(x.double(), weight.double().t()).float()
    shape = (1,) * (rank - 1) + (k,)
    strides = ((0 if zero_stride else k),) * (rank - 1) + (1,)
    return x.cuda().as_strided(shape, strides), weight.cuda(), expected.view(*shape[:-1], n)


def check(actual, x, weight, expected, saved):
    assert actual.shape == expected.shape and actual.dtype == x.dtype and actual.device == x.device
    assert actual.is_contiguous()
    assert actual.untyped_storage().data_ptr() not in (x.untyped_storage().data_ptr(),
                                                       weight.untyped_storage().data_ptr())
    error = row_errors(actual.float().cpu().reshape(1, -1), expected.reshape(1, -1))
    assert (max(error["relative_l2"], error["peak_relative"]) <= LIMITS[x.dtype]
            or error["max_abs"] <= ABS_LIMITS[x.dtype]), error
    assert all(torch.equal(a.cpu(), b) for a, b in zip((x, weight), saved))


@torch.inference_mode()
def test_profiled_geometries_against_an_independent_control(gpu_ops):
    from xinfer_amd.projection_gemv import projection_gemv

    for dtype in DTYPES:
        for index, (n, k) in enumerate(SHAPES):
            log(f"projection gemv {dtype} n={n} k={k}")
            x, weight, expected = inputs(n, k, dtype, rank=3, zero_stride=index != 2)
            saved = [x.cpu(), weight.cpu()]
            check(projection_gemv(x, weight), x, weight, expected, saved)


@torch.inference_mode()
def test_masked_tails_and_exact_bfloat16_rounding(gpu_ops):
    from xinfer_amd.projection_gemv import projection_gemv

    for dtype in DTYPES:
        for k in (33, 2049, 1024):
            log(f"projection gemv binary {dtype} k={k}")
            x, weight, expected = inputs(7, k, dtype, binary=True, zero_stride=True)
            saved = [x.cpu(), weight.cpu()]
            actual = projection_gemv(x, weight)
            check(actual, x, weight, expected, saved)
            assert torch.equal(actual.cpu(), expected.to(dtype))
            x.zero_()
            check(projection_gemv(x, weight), x, weight, torch.zeros_like(expected), [x.cpu(), weight.cpu()])


@torch.inference_mode()
def test_offset_singleton_layouts_repeats_and_nondefault_stream(gpu_ops):
    from xinfer_amd.projection_gemv import projection_gemv

    for dtype in DTYPES:
        for rank in (2, 3):
            for zero_stride in (False, True):
                log(f"projection gemv offset {dtype} rank={rank} zero_stride={zero_stride}")
                x, weight, expected = inputs(17, 2048, dtype, rank=rank)
                backing = torch.empty(2049, device="cuda", dtype=dtype)
                backing[1:].copy_(x.reshape(-1))
                strides = ((0 if zero_stride else 2048),) * (rank - 1) + (1,)
                x = backing[1:].as_strided(x.shape, strides)
                saved = [x.cpu(), weight.cpu()]
                stream = torch.cuda.Stream()
                stream.wait_stream(torch.cuda.current_stream())
                with torch.cuda.stream(stream):
                    actual = projection_gemv(x, weight)
                    repeat = projection_gemv(x, weight)
                stream.synchronize()
                check(actual, x, weight, expected, saved)
                assert torch.equal(actual, repeat)
                assert actual.untyped_storage().data_ptr() != repeat.untyped_storage().data_ptr()


@torch.inference_mode()
def test_reference_error_messages(gpu_ops):
    from xinfer_amd.projection_gemv import projection_gemv

    x = torch.randn(1, 64, device="cuda", dtype=torch.bfloat16)
    w = torch.randn(8, 64, device="cuda", dtype=torch.bfloat16)
    cases = [
        ((x.cpu(), w), "colocated CUDA tensors"),
        ((x.half(), w.half()), "matching BF16 or FP32"),
        ((x.float(), w), "matching BF16 or FP32"),
        ((torch.randn(2, 64, device="cuda", dtype=torch.bfloat16), w), "one input row and a 2D weight"),
        ((x[0], w), "one input row and a 2D weight"),
        ((x, w[:, :32]), "matching contiguous reduction dimensions"),
        ((x, w.t().contiguous().t()), "matching contiguous reduction dimensions"),
        ((x[:, :0], w[:, :0]), "positive dimensions"),
    ]
    for args, message in cases:
        with pytest.raises(ValueError, match=message):
            projection_gemv(*args)
    torch.library.opcheck(torch.ops.xinfer.projection_gemv.default, (x, w),
                          test_utils=("test_schema", "test_faketensor"))
