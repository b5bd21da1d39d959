"""The C-ABI library loads and exports every symbol include/aspire_hip.h declares (no GPU calls)."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "aspire_hip.h"
LIB = ROOT / "aspire_amd" / "libaspire_hip.so"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(aspire_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_python_binding_set():
    from aspire_amd import _lib

    assert declared_functions() == sorted(_lib.EXPORTED)


@pytest.mark.skipif(not LIB.exists(), reason="libaspire_hip.so not built")
def test_library_exports_every_declared_symbol():
    import torch  # noqa: F401  (binds the HIP runtime torch ships)

    lib = ctypes.CDLL(str(LIB))
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, missing
    lib.aspire_build_info.restype = ctypes.c_char_p
    info = lib.aspire_build_info().decode()
    assert "gfx950" in info and "sources_sha256=" in info
    lib.aspire_max_kv_tile.restype = ctypes.c_int32
    assert lib.aspire_max_kv_tile() == 16
