"""AOTInductor packages that carry the native attention library.

The package-embedding step of the reference (compiler/common/package.py:36-86)
for this PyTorch (2.10, ROCm): the same ``compile_package`` entry point,
arguments and preflight errors, so the exporter calls it unchanged.

* The wrapper is compiled with the operators' C shims
  (``aot_inductor.custom_ops_to_c_shims``) and linked against each native
  library by its ``lib<name>.so`` name, with a ``$ORIGIN`` run path, so the
  wrapper calls ``aoti_torch_cuda_flash_attention`` and friends directly.
* The libraries go into the package next to the wrapper.  This PyTorch's
  package writer accepts one shared object per model, and its loader takes the
  last shared object of the model directory as the model, so each library is
  written into the model directory ahead of the wrapper's shared object.
  Loading extracts the directory, the dynamic linker finds the library through
  ``$ORIGIN``, and its static initialisers register the operators: the package
  needs no ``torch.ops.load_library``.

``load_package`` is ``torch._inductor.aoti_load_package`` for a fresh
process: in this PyTorch the loader needs ``torch._inductor.codecache``
imported first.
"""

from __future__ import annotations

from contextlib import contextmanager
import os
from pathlib import Path
import zipfile

from .attention import require

LINK_VARIABLES = ("LIBRARY_PATH", "LD_RUN_PATH")


@contextmanager
def linking_environment(libraries):
    """Point the linker at the libraries' directories and request a $ORIGIN run path.

    The variables are process-wide (Inductor's config patches are per thread),
    so their previous values are restored on exit, also after a failure.
    """
    if not libraries:
        yield
        return
    saved = {name: os.environ.get(name) for name in LINK_VARIABLES}
    search = [str(Path(library).parent) for library in libraries]
    if saved["LIBRARY_PATH"]:
        search.append(saved["LIBRARY_PATH"])
    os.environ["LIBRARY_PATH"] = os.pathsep.join(dict.fromkeys(search))
    os.environ["LD_RUN_PATH"] = "$ORIGIN"
    try:
        yield
    finally:
        for name, value in saved.items():
            if value is None:
                os.environ.pop(name, None)
            else:
                os.environ[name] = value


def checked_libraries(native_libraries):
    """Resolved library paths, after the reference's preflight checks."""
    libraries = [Path(path).resolve() for path in native_libraries]
    require(all(path.is_file() for path in libraries), "Native operator library is missing")
    require(len({path.name for path in libraries}) == len(libraries), "Duplicate native library name")
    require(
        all(path.name.startswith("lib") and path.name.endswith(".so") for path in libraries),
        "Expected a native library named lib<name>.so",
    )
    return libraries


def embed_libraries(package, libraries):
    """Rewrite `package` with each library in the model directory, ahead of the wrapper .so."""
    package = Path(package)
    staged = package.with_name(package.name + ".partial")
    with zipfile.ZipFile(package) as source:
        entries = source.infolist()
        wrappers = [entry.filename for entry in entries if entry.filename.endswith(".wrapper.so")]
        require(len(wrappers) == 1, "Expected one compiled wrapper in the package")
        model_dir = wrappers[0].rsplit("/", 1)[0]
        with zipfile.ZipFile(staged, "w", zipfile.ZIP_STORED) as target:
            for entry in entries:
                if entry.filename == wrappers[0]:
                    for library in libraries:
                        target.write(library, arcname=f"{model_dir}/{Path(library).name}")
                target.writestr(entry, source.read(entry.filename))
    os.replace(staged, package)


def compile_package(exported, destination, *, inductor_configs, native_libraries=(), custom_op_shims=None):
    """AOT-compile `exported` into the package `destination` (reference: package.py:36-86)."""
    import torch

    if not native_libraries and not custom_op_shims:
        return torch._inductor.aoti_compile_and_package(
            exported, package_path=str(destination), inductor_configs=inductor_configs
        )
    libraries = checked_libraries(native_libraries)

    from torch._inductor import config
    from torch._inductor.package import package_aoti

    shims = dict(config.aot_inductor.custom_ops_to_c_shims)
    shims.update(custom_op_shims or {})
    link = list(config.aot_inductor.custom_op_libs or [])
    link += [path.name[len("lib") : -len(".so")] for path in libraries]
    args, kwargs = exported.example_inputs
    patches = {
        "aot_inductor.custom_ops_to_c_shims": shims,
        "aot_inductor.custom_op_libs": list(dict.fromkeys(link)),
    }
    with config.patch(patches), linking_environment(libraries):
        files = torch._inductor.aot_compile(
            exported.module(), args, kwargs, options={**inductor_configs, "aot_inductor.package": True}
        )
    package_aoti(str(destination), files)
    embed_libraries(destination, libraries)
    return str(destination)


def load_package(path):
    """Load a package in any process (see the module docstring)."""
    import torch
    import torch._inductor.codecache  # noqa: F401  (needed by this PyTorch's loader)

    return torch._inductor.aoti_load_package(str(path))
