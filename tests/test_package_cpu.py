"""Package-embedding step without a GPU: preflight errors, the linker
environment, and where the native library lands in the archive.

Counterpart of compiler/common/tests/test_package.py:133-183 (PackagePreflight).
"""

import os
from pathlib import Path
import subprocess
from unittest.mock import patch, sentinel
import zipfile

import pytest
import torch

from xinfer_amd.package import compile_package, embed_libraries, linking_environment


def test_invalid_libraries_fail_before_compilation_or_output(tmp_path):
    invalid = tmp_path / "attention.so"
    invalid.touch()
    duplicates = []
    for part in ("one", "two"):
        (tmp_path / part).mkdir()
        duplicates.append(tmp_path / part / "libattention.so")
        duplicates[-1].touch()
    destination = tmp_path / "model.pt2"
    for selected, message in (
        ([tmp_path / "libmissing.so"], "Native operator library is missing"),
        ([invalid], "Expected a native library named"),
        (duplicates, "Duplicate native library name"),
    ):
        with patch.object(torch._inductor, "aot_compile") as compile, pytest.raises(ValueError, match=message):
            compile_package(sentinel.exported, destination, inductor_configs={}, native_libraries=selected)
        compile.assert_not_called()
        assert not destination.exists()


def test_link_environment_restores_existing_values_after_failure():
    original = {"LIBRARY_PATH": "/existing/lib", "LD_RUN_PATH": "/existing/run"}
    with patch.dict(os.environ, original):
        with pytest.raises(RuntimeError, match="compile failed"):
            with linking_environment([Path("/build/libattention.so")]):
                assert os.environ["LIBRARY_PATH"] == "/build" + os.pathsep + "/existing/lib"
                assert os.environ["LD_RUN_PATH"] == "$ORIGIN"
                raise RuntimeError("compile failed")
        for name, value in original.items():
            assert os.environ[name] == value


def test_link_environment_restores_absent_values():
    with patch.dict(os.environ):
        os.environ.pop("LIBRARY_PATH", None)
        os.environ.pop("LD_RUN_PATH", None)
        with linking_environment([Path("/build/libattention.so")]):
            assert os.environ["LIBRARY_PATH"] == "/build"
            assert os.environ["LD_RUN_PATH"] == "$ORIGIN"
        assert "LIBRARY_PATH" not in os.environ
        assert "LD_RUN_PATH" not in os.environ


def test_library_is_found_by_name_and_never_unloaded(library_path):
    """Packages name the library by its SONAME, so a process resolves every
    package to one loaded copy; the library is NODELETE because its operator
    registrations and the Python handles to them must outlive a dropped package."""
    dynamic = subprocess.check_output(["readelf", "-d", str(library_path)], text=True)
    assert f"Library soname: [{library_path.name}]" in dynamic
    flags = [line for line in dynamic.splitlines() if "FLAGS_1" in line]
    assert flags and "NODELETE" in flags[0]


def test_library_is_written_ahead_of_the_wrapper_in_the_model_directory(tmp_path):
    """The package loader of this PyTorch takes the model directory's last
    shared object as the model, so the library must precede the wrapper."""
    package = tmp_path / "model.pt2"
    members = {
        "model/archive_format": b"pt2",
        "model/data/aotinductor/model/abc.wrapper.cpp": b"// wrapper",
        "model/data/aotinductor/model/abc.wrapper.so": b"\x7fELF wrapper",
        "model/data/aotinductor/model/abc.wrapper_metadata.json": b"{}",
    }
    with zipfile.ZipFile(package, "w") as archive:
        for name, data in members.items():
            archive.writestr(name, data)
    library = tmp_path / "libxinfer_attention_ops.so"
    library.write_bytes(b"\x7fELF library")
    embed_libraries(package, [library])
    with zipfile.ZipFile(package) as archive:
        names = archive.namelist()
        assert names == [
            "model/archive_format",
            "model/data/aotinductor/model/abc.wrapper.cpp",
            "model/data/aotinductor/model/libxinfer_attention_ops.so",
            "model/data/aotinductor/model/abc.wrapper.so",
            "model/data/aotinductor/model/abc.wrapper_metadata.json",
        ]
        for name, data in members.items():
            assert archive.read(name) == data
        assert archive.read("model/data/aotinductor/model/libxinfer_attention_ops.so") == library.read_bytes()
        shared = [name for name in names if name.startswith("model/data/aotinductor/model/") and name.endswith(".so")]
        assert shared[-1].endswith(".wrapper.so")
    assert not package.with_name(package.name + ".partial").exists()
