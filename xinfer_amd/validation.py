"""The attention library a bundle carries, loaded for the eager validation stage.

Counterpart of tools/validation/common/attention.py:14-51.  xinfer's
validation chain runs the adapted model eagerly before it runs the AOTI
packages, and the eager stage must use the operator the packages embed, not
whatever build happens to be on disk.  ``load_packaged_attention_ops(bundle)``
therefore:

* returns the library already registered in this process, if any (the
  package loaders register it themselves when they load a package);
* otherwise reads the one ``libxinfer_attention_ops.so`` stored under
  ``data/aotinductor/`` in the bundle's ``prefill.pt2``, writes it to a
  private temporary directory that lives as long as the process, and loads it
  with ``load_attention_ops`` (which also registers the fakes).

A bundle without exactly one such library, or with an empty one, is rejected
with ``ValueError``, as in the reference.
"""

from __future__ import annotations

from pathlib import Path
import tempfile
import zipfile

from . import attention

_extracted = None  # the temporary directory holding the extracted library


def packaged_attention_library(package):
    """Bytes of the attention library stored in an AOTI package (a .pt2 zip)."""
    suffix = "/" + attention.ATTENTION_LIBRARY
    with zipfile.ZipFile(package) as archive:
        entries = [name for name in archive.namelist() if "/data/aotinductor/" in name and name.endswith(suffix)]
        attention.require(len(entries) == 1, "Package is missing its attention library; re-export both entries")
        payload = archive.read(entries[0])
    attention.require(len(payload) > 0, "Packaged attention library is empty")
    return payload


def load_packaged_attention_ops(packages):
    """Register the attention operators of the bundle directory ``packages``; returns the library path."""
    global _extracted
    if attention._loaded is not None:
        return attention.attention_library()
    payload = packaged_attention_library(Path(packages) / "prefill.pt2")
    directory = tempfile.TemporaryDirectory(prefix="xinfer-attention-")
    library = Path(directory.name) / attention.ATTENTION_LIBRARY
    library.write_bytes(payload)
    try:
        attention.load_attention_ops(library)
    except Exception:
        directory.cleanup()
        raise
    _extracted = directory
    return library
