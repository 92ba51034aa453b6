"""The CMake target builds the same library (CPU: hipcc cross-compiles for gfx950).

Counterpart of the reference's operator target
(compiler/common/kernels/CMakeLists.txt:1-7, added by the top-level
CMakeLists.txt with find_package(Torch)): xinfer_amd/csrc/CMakeLists.txt is
configured with Ninja against this PyTorch and built into a temporary
directory.  The library must carry gfx950 device code, keep the SONAME the
reference's loaders and validator look for, and export every function that
include/*.h declares; a fresh process loads it (registering the operators)
without a GPU.
"""

import json
from pathlib import Path
import shutil
import subprocess
import sys
import textwrap

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIP_COMPILER = Path("/opt/rocm/lib/llvm/bin/clang++")


@pytest.fixture(scope="module")
def cmake_library(tmp_path_factory):
    if shutil.which("cmake") is None or shutil.which("ninja") is None or not HIP_COMPILER.exists():
        pytest.skip("cmake, ninja and ROCm clang are needed for the CMake build")
    import torch

    build = tmp_path_factory.mktemp("cmake_build")
    subprocess.run(["cmake", "-S", str(ROOT / "xinfer_amd" / "csrc"), "-B", str(build), "-G", "Ninja",
                    f"-DCMAKE_PREFIX_PATH={torch.utils.cmake_prefix_path}", f"-DCMAKE_HIP_COMPILER={HIP_COMPILER}"],
                   check=True, capture_output=True, text=True, timeout=600)
    subprocess.run(["cmake", "--build", str(build), "-j", "8"], check=True, capture_output=True, text=True,
                   timeout=1200)
    library = build / "libxinfer_attention_ops.so"
    assert library.is_file()
    return library


def test_cmake_library_carries_gfx950_code_and_the_soname(cmake_library):
    data = cmake_library.read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    dynamic = subprocess.check_output(["readelf", "-d", str(cmake_library)], text=True)
    assert "Library soname: [libxinfer_attention_ops.so]" in dynamic
    assert "Shared library: [libtorch.so]" in dynamic


LOADER = textwrap.dedent(
    """
    import ctypes, json, sys
    sys.path.insert(0, sys.argv[1])
    sys.path.insert(0, sys.argv[1] + '/tests')
    from test_library_cpu import declared_functions
    import torch
    lib = ctypes.CDLL(sys.argv[2])
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    lib.xinfer_status_string.restype = ctypes.c_char_p
    print(json.dumps(dict(missing=missing, declared=len(declared_functions()),
                          registered=hasattr(torch.ops.xinfer, 'batched_flash_attention'),
                          message=lib.xinfer_status_string(6).decode())))
    """
)


def test_cmake_library_exports_every_declared_function(cmake_library):
    result = subprocess.run([sys.executable, "-c", LOADER, str(ROOT), str(cmake_library)], capture_output=True,
                            text=True, timeout=300)
    assert result.returncode == 0, result.stderr[-3000:]
    report = json.loads(result.stdout.splitlines()[-1])
    assert report["declared"] > 10 and report["missing"] == []
    assert report["registered"]
    assert report["message"] == "Invalid valid-prefix length"
