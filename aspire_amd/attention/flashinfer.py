"""Build identity and tile-size helpers (HIP implementation).

Drop-in for ``aspire/attention/flashinfer.py``. The reference validates that the
installed FlashInfer carries its persistent-attention patch
(flashinfer.py:14-60), sizes the logits-dump stride padding from FlashInfer's
KV tile (flashinfer.py:63-105) and names the attention backend
(flashinfer.py:108-117). Here the attention kernels are this package's own
HIP library, so validation reports that library's build identity, the tile is
the kernel's 16-token page step, and the backend name is ``"hip"``.
"""

from __future__ import annotations

import functools
import hashlib
from pathlib import Path

import torch

from aspire_amd import _lib

FLASHINFER_COMMIT = None
FLASHINFER_PATCH_SHA256 = None


def validate_flashinfer_patch(csrc_dir: str | Path | None = None,
                              include_dir: str | Path | None = None) -> dict:
    """Fail early when the HIP library is absent; return its build identity.

    Same dict keys as the reference (flashinfer.py:56-60). Raises RuntimeError
    when libaspire_hip.so cannot be loaded. The directory arguments are
    accepted for signature compatibility and ignored.
    """
    info = _lib.build_info()
    return {
        "expected_commit": "libaspire_hip",
        "patch_sha256": hashlib.sha256(info.encode()).hexdigest(),
        "installed_sources_sha256": info.split("sources_sha256=", 1)[-1].split(" ", 1)[0],
    }


def compute_max_cta_tile_kv(head_dim_qk: int = 128, head_dim_vo: int = 128, dtype_bytes: int = 2,
                            device: int = 0) -> int:
    """KV tile of the HIP attention kernel (tokens), used as the dump-stride pad multiple.

    The kernel writes dump entries only for ``kv_idx < kv_len``, so padding is
    not needed for safety; returning the real tile keeps the reference's
    stride arithmetic (base.py:314-320) meaningful.
    """
    return int(_lib.lib().aspire_max_kv_tile())


@functools.lru_cache(maxsize=None)
def _resolve_flashinfer_attention_backend(device_index: int, dtype: torch.dtype) -> str:
    return "hip"


def resolve_flashinfer_attention_backend(dtype: torch.dtype) -> str:
    if not torch.cuda.is_available():
        raise RuntimeError("attention backend resolution requires a ROCm GPU.")
    return _resolve_flashinfer_attention_backend(torch.cuda.current_device(), dtype)
