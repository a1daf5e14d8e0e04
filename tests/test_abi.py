"""The C-ABI library loads on the CPU host and exports every symbol that
include/zoomkv_gfx950.h declares (no compute calls: no GPU here)."""
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def _declared():
    text = (ROOT / "include" / "zoomkv_gfx950.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(zkv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = _declared()
    assert "zkv_kivi4_decode_attention" in names and "zkv_last_error" in names


def test_library_exports_every_declared_symbol():
    from zoomkv_revision_amd import _lib
    L = _lib.lib()
    for name in _declared():
        assert hasattr(L, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert L.zkv_version().decode().startswith("zoomkv_gfx950")
    assert L.zkv_last_error() == b""


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    import pytest
    from zoomkv_revision_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(_lib.ZkvError):
        _lib.lib()
