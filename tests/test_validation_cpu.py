"""The eager-validation loader takes the attention library out of a bundle (CPU).

Counterpart of the reference's packaged-operator selection
(tools/validation/common/attention.py:14-51).  The packages here are zip
archives laid out like AOTI packages; the GPU package tests check the same
loader on real ones.
"""

import json
from pathlib import Path
import subprocess
import sys
import textwrap
import zipfile

import pytest

from xinfer_amd import validation

ROOT = Path(__file__).resolve().parents[1]
ENTRY = "prefill/data/aotinductor/model/libxinfer_attention_ops.so"


def write_package(path, entries):
    with zipfile.ZipFile(path, "w") as archive:
        for name, payload in entries.items():
            archive.writestr(name, payload)
    return path


def test_payload_is_the_one_packaged_library(tmp_path, library_path):
    payload = library_path.read_bytes()
    package = write_package(tmp_path / "prefill.pt2", {ENTRY: payload, "prefill/data/aotinductor/model/x.wrapper.so": b"w"})
    assert validation.packaged_attention_library(package) == payload


@pytest.mark.parametrize(
    "entries,message",
    [
        ({"prefill/data/aotinductor/model/other.so": b"x"}, "missing its attention library"),
        ({ENTRY: b"x", "prefill/data/aotinductor/extra/libxinfer_attention_ops.so": b"y"},
         "missing its attention library"),
        ({"prefill/libxinfer_attention_ops.so": b"x"}, "missing its attention library"),
        ({ENTRY: b""}, "library is empty"),
    ],
)
def test_malformed_packages_are_rejected(tmp_path, entries, message):
    package = write_package(tmp_path / "prefill.pt2", entries)
    with pytest.raises(ValueError, match=message):
        validation.packaged_attention_library(package)


WORKER = textwrap.dedent(
    """
    import json, sys
    sys.path.insert(0, sys.argv[1])
    import torch
    from xinfer_amd import attention, validation
    library = validation.load_packaged_attention_ops(sys.argv[2])
    again = validation.load_packaged_attention_ops(sys.argv[2])
    print(json.dumps(dict(library=str(library), again=str(again),
                          registered=hasattr(torch.ops.xinfer, 'batched_flash_attention'),
                          bytes=library.stat().st_size)))
    """
)


def test_fresh_process_loads_the_extracted_library(tmp_path, library_path):
    bundle = tmp_path / "bundle"
    bundle.mkdir()
    write_package(bundle / "prefill.pt2", {ENTRY: library_path.read_bytes()})
    result = subprocess.run([sys.executable, "-c", WORKER, str(ROOT), str(bundle)], capture_output=True,
                            text=True, timeout=300)
    assert result.returncode == 0, result.stderr[-3000:]
    report = json.loads(result.stdout.splitlines()[-1])
    assert report["registered"]
    assert report["library"] == report["again"]  # the registered library is reused
    assert Path(report["library"]).name == "libxinfer_attention_ops.so"
    assert not report["library"].startswith(str(ROOT))
    assert report["bytes"] == library_path.stat().st_size
