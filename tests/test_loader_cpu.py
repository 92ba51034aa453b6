"""Library selection of xinfer_amd.attention.load_attention_ops, with a stand-in torch.

Mirrors the reference's loader tests (compiler/common/tests/test_native_library.py:
explicit library, environment override, model default, missing library, one
library per process) without touching the real operator registry.
"""

import os
from types import SimpleNamespace
from unittest.mock import Mock, patch

import pytest

from xinfer_amd import attention


@pytest.fixture
def fake_env(tmp_path, monkeypatch):
    library = tmp_path / "selected build" / "libxinfer_attention_ops.so"
    library.parent.mkdir()
    library.touch()
    monkeypatch.delenv("XINFER_ATTENTION_OPS_LIBRARY", raising=False)
    monkeypatch.setattr(attention, "_loaded", None)
    default = tmp_path / "lib" / "libxinfer_attention_ops.so"
    monkeypatch.setattr(attention, "ROOT", tmp_path)
    fake_torch = SimpleNamespace(
        ops=SimpleNamespace(load_library=Mock(), xinfer=SimpleNamespace()),
        library=SimpleNamespace(register_fake=Mock(return_value=lambda function: function)),
    )
    return SimpleNamespace(library=library.resolve(), default=default, torch=fake_torch, root=tmp_path)


def test_explicit_library_registers_the_flash_fake(fake_env):
    with patch.dict("sys.modules", {"torch": fake_env.torch}):
        attention.load_attention_ops(fake_env.library)
    fake_env.torch.ops.load_library.assert_called_once_with(str(fake_env.library))
    names = [call.args[0] for call in fake_env.torch.library.register_fake.call_args_list]
    # The stand-in registry exposes no operators, so only the unconditional fake is registered.
    assert names == ["xinfer::flash_attention"]
    assert attention.attention_library() == fake_env.library


def test_missing_default_library_raises_file_not_found(fake_env):
    with patch.dict("sys.modules", {"torch": None}), pytest.raises(FileNotFoundError) as error:
        attention.load_attention_ops(model="qwen3")
    assert str(fake_env.default) in str(error.value)
    assert attention._loaded is None


def test_model_default_and_environment_override(fake_env, monkeypatch):
    fake_env.default.parent.mkdir(parents=True)
    fake_env.default.touch()
    with patch.dict("sys.modules", {"torch": fake_env.torch}):
        attention.load_attention_ops(model="qwen35")
    fake_env.torch.ops.load_library.assert_called_once_with(str(fake_env.default))
    monkeypatch.setattr(attention, "_loaded", None)
    monkeypatch.setenv("XINFER_ATTENTION_OPS_LIBRARY", str(fake_env.library))
    with patch.dict("sys.modules", {"torch": fake_env.torch}):
        attention.load_attention_ops(model="qwen3")
    assert attention._loaded == fake_env.library


def test_selection_errors(fake_env):
    with pytest.raises(ValueError, match="Select a model"):
        attention.load_attention_ops()
    with pytest.raises(ValueError, match="Unknown model"):
        attention.load_attention_ops(model="llama")
    with pytest.raises(ValueError, match="Load the native attention library"):
        attention.attention_library()
    with patch.dict("sys.modules", {"torch": fake_env.torch}):
        attention.load_attention_ops(fake_env.library)
        attention.load_attention_ops()  # already loaded: no-op
        other = fake_env.root / "libother.so"
        other.touch()
        with pytest.raises(ValueError, match="two different attention libraries"):
            attention.load_attention_ops(other)
    assert fake_env.torch.ops.load_library.call_count == 1


def test_cache_extent_carries_only_a_length():
    extent = attention.cache_extent(1024)
    assert extent.shape == (1025,) and str(extent.dtype) == "torch.uint8" and extent.device.type == "cpu"
