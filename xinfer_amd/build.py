"""Build libxinfer_attention_ops.so for gfx950 with hipcc, in-tree.

The library holds the HIP kernels, the C ABI of include/xinfer_attention.h and
the torch.library / AOTInductor registration layer (replacing the CMake target
of the reference, compiler/common/kernels/CMakeLists.txt:1-7).  It links
against the HIP runtime that ships inside torch so one runtime serves the
process, and carries an RPATH to torch's library directory.

    python -m xinfer_amd.build [--verbose]
"""

from __future__ import annotations

import argparse
import concurrent.futures
import os
from pathlib import Path
import shutil
import subprocess
import sysconfig

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
LIB_DIR = PACKAGE / "lib"
OBJ_DIR = PACKAGE / "_build"
LIBRARY_NAME = "libxinfer_attention_ops.so"
ARCH = "gfx950"

KERNEL_SOURCES = ("append.hip", "decode.hip", "prefill.hip", "prefill_d256.hip", "merge.hip", "norm_rope.hip",
                  "gemv.hip", "scratch.hip")
HOST_SOURCES = ("capi.cpp",)
TORCH_SOURCES = ("torch_ops.cpp",)

# Packed fp32 VALU instructions are kept out of every device build.
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

# Per-source scheduling strategies: they reorder the same instructions (the
# results are bit for bit those of the default scheduler).  Measured on
# MI355X: max-ilp takes the head-dim-256 prefill from 535 to 516 us (cfg5) and
# the decode kernels 1-2 % faster; iterative-ilp takes the head-dim-64/128
# prefill from 21.4 to 20.8 us (cfg2), where max-ilp gained nothing, and made
# the head-dim-256 kernel 8 % slower.  max-ilp also takes the fused
# norm/RoPE/append kernel from 4.97 to 4.85 us at cfg2's 512 tokens.
SOURCE_FLAGS = {
    "decode.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "norm_rope.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "prefill.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
    "prefill_d256.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
}


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise FileNotFoundError("hipcc not found; ROCm is required to build the attention library")
    return found


def rocm_path() -> Path:
    return Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def torch_paths():
    import torch
    from torch.utils import cpp_extension

    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    includes = cpp_extension.include_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return torch_lib, includes, abi


def _run(command, verbose):
    if verbose:
        print(" ".join(map(str, command)), flush=True)
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(
            f"command failed ({result.returncode}): {' '.join(map(str, command))}\n"
            f"{result.stdout}\n{result.stderr}"
        )


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link the library; returns its path."""
    compiler = hipcc()
    torch_lib, torch_includes, abi = torch_paths()
    OBJ_DIR.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    common = ["-O3", "-fPIC", "-std=c++17", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
    # Host-only translation units still use the HIP runtime API headers.
    host = [f"-isystem{rocm_path() / 'include'}", "-D__HIP_PLATFORM_AMD__"]
    # MFMA accumulators in VGPRs: left to its heuristics, the compiler put the
    # D = 256 prefill accumulators in AGPRs and copied all 128 of them to
    # VGPRs and back on every tile.
    device = [f"--offload-arch={ARCH}", *NO_PACKED_FP32, "-ffp-contract=fast", "-mllvm", "-amdgpu-mfma-vgpr-form=1"]
    torch_flags = [f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *(f"-isystem{p}" for p in torch_includes),
                   f"-isystem{sysconfig.get_paths()['include']}", "-DTORCH_EXTENSION_NAME=xinfer_attention_ops",
                   # torch is built with GCC: keep the Itanium mangling GCC uses for constrained templates.
                   "-fclang-abi-compat=17"]
    jobs_list = []
    for name in KERNEL_SOURCES:
        jobs_list.append([compiler, "-x", "hip", *common, *device, *SOURCE_FLAGS.get(name, []), "-c", CSRC / name,
                          "-o", OBJ_DIR / f"{name}.o"])
    for name in HOST_SOURCES:
        jobs_list.append([compiler, "-x", "c++", *common, *host, "-c", CSRC / name, "-o", OBJ_DIR / f"{name}.o"])
    for name in TORCH_SOURCES:
        jobs_list.append(
            [compiler, "-x", "c++", *common, *host, *torch_flags, "-Wno-unused-parameter", "-c", CSRC / name,
             "-o", OBJ_DIR / f"{name}.o"]
        )
    workers = jobs or min(8, os.cpu_count() or 1)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for future in [pool.submit(_run, job, verbose) for job in jobs_list]:
            future.result()
    objects = [OBJ_DIR / f"{name}.o" for name in (*KERNEL_SOURCES, *HOST_SOURCES, *TORCH_SOURCES)]
    output = LIB_DIR / LIBRARY_NAME
    temporary = output.with_suffix(".so.tmp")
    # -z nodelete: the operators are registered with the process-wide
    # dispatcher, and Python keeps handles to them (torch.ops.xinfer.*), so the
    # library stays mapped after the last dlclose, e.g. when the AOTInductor
    # package that brought it in is dropped and another one is loaded later.
    _run(
        [compiler, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objects, "-o", temporary,
         f"-L{torch_lib}", "-ltorch", "-ltorch_cpu", "-ltorch_hip", "-lc10", "-lc10_hip", "-lamdhip64",
         f"-Wl,-rpath,{torch_lib}", f"-Wl,-soname,{LIBRARY_NAME}", "-Wl,--no-undefined", "-Wl,-z,nodelete"],
        verbose,
    )
    os.replace(temporary, output)
    return output


def library_path() -> Path:
    return LIB_DIR / LIBRARY_NAME


def main():
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--verbose", action="store_true")
    args = parser.parse_args()
    print(build(verbose=args.verbose))


if __name__ == "__main__":
    main()
