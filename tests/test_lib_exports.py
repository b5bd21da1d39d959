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


@pytest.mark.skipif(not LIB.exists(), reason="libaspire_hip.so not built")
@pytest.mark.parametrize("scale", [float("nan"), float("inf"), -0.1, 0.0, 1e31])
def test_prefill_rejects_bad_sm_scale_on_the_host(scale):
    """The prefill entry checks sm_scale before anything reaches the GPU (so this runs without
    one): NaN, infinities, non-positive and huge scales are refused with a clear error."""
    import torch  # noqa: F401

    from aspire_amd import _lib

    a = _lib.PrefillArgs()
    a.num_qo_heads, a.num_kv_heads, a.head_dim, a.page_size = 32, 8, 128, 16
    a.block_tokens = _lib.lib().aspire_prefill_block_tokens(32, 8)
    a.num_rows, a.total_blocks = 1, 1
    a.cache_stride_p, a.cache_stride_t = 2 * 16 * 8 * 128, 8 * 128
    a.sm_scale = scale
    rc = _lib.lib().aspire_prefill_run(ctypes.byref(a), None)
    assert rc == _lib.ASPIRE_ERR_INVALID
    assert "sm_scale" in _lib.lib().aspire_last_error().decode()
