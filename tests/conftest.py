"""Shared pytest configuration for the xinfer attention tests.

Tests marked ``gpu`` need an MI355X (ROCm torch with a visible device) and the
built library; they fail loudly -- never fall back -- when the library is
missing.  Everything else runs on the CPU.
"""

from pathlib import Path
import sys

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU and the built HIP library")


@pytest.fixture(scope="session")
def library_path():
    from xinfer_amd.build import library_path as path

    library = path()
    if not library.is_file():
        raise FileNotFoundError(f"Build the native attention library first: {library}")
    return library


@pytest.fixture(scope="session")
def gpu_ops(library_path):
    """Load the operators for GPU tests; a missing GPU is an error, not a skip."""
    import torch

    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a visible AMD GPU")
    from xinfer_amd.attention import load_attention_ops

    load_attention_ops(library_path)
    return torch.ops.xinfer
