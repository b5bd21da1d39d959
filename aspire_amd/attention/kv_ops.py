"""Torch custom operators for paged KV-cache writes (HIP implementation).

Drop-in for ``aspire/attention/kv_ops.py``: the same operator names and schemas,
``mylib::update_kv`` (kv_ops.py:12-60) and ``mylib::update_kv_padded``
(kv_ops.py:127-187), both mutating ``kv_cache`` in place with fake (meta)
implementations for ``torch.compile``. Each call is one launch of the fused
append kernel in libaspire_hip.so (``aspire_paged_kv_append``), which folds in
FlashInfer's ``get_seq_lens`` and ``get_batch_indices_positions`` (the reference
runs three launches). The kernel skips padding tokens exactly as
kv_ops.py:92-98 does, so both operators share it; the reference's unpadded
``update_kv`` only ever sees inputs where every token belongs to a row.
"""

from __future__ import annotations

import torch

from aspire_amd import _lib

_SCHEMA = (
    "(Tensor k, Tensor v, Tensor kv_append_indptr, Tensor(a!) kv_cache, "
    "Tensor kv_page_indices, Tensor kv_page_indptr, Tensor kv_last_page_len, "
    "int page_size) -> ()"
)


def _i32(t: torch.Tensor) -> torch.Tensor:
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def paged_kv_append(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_last_page_len,
                    page_size: int) -> None:
    """Scatter ``k``/``v`` ``[T, H_kv, D]`` into ``kv_cache`` ``[P, 2, page, H_kv, D]``."""
    total_tokens = k.shape[0]
    if total_tokens == 0:
        return
    _lib.require_cuda(k, v, kv_cache, kv_append_indptr, kv_page_indices, what="update_kv_padded")
    head_dim = k.shape[2]
    num_heads = k.shape[1]
    if k.stride(-1) != 1 or v.stride(-1) != 1:
        raise ValueError("update_kv_padded requires contiguous k/v head dimensions")
    if k.stride(1) != head_dim or v.stride(1) != head_dim:
        raise ValueError("update_kv_padded requires contiguous k/v heads")
    if kv_cache.stride(-1) != 1:
        raise ValueError("update_kv_padded requires a contiguous cache head dimension")
    if k.dtype != kv_cache.dtype or v.dtype != kv_cache.dtype or kv_cache.element_size() != 2:
        raise ValueError("k, v and kv_cache must share a 16-bit dtype")
    num_seq = kv_last_page_len.shape[0]
    if kv_page_indptr.shape[0] < num_seq + 1 or kv_append_indptr.shape[0] < num_seq + 1:
        raise ValueError("kv_page_indptr and kv_append_indptr need len(kv_last_page_len) + 1 entries")
    ai, pi, pp, lp = (_i32(kv_append_indptr), _i32(kv_page_indices), _i32(kv_page_indptr),
                      _i32(kv_last_page_len))
    L = _lib.lib()
    rc = L.aspire_paged_kv_append(
        _lib.ptr(k), _lib.ptr(v), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        _lib.ptr(ai), _lib.ptr(pi), _lib.ptr(pp), _lib.ptr(lp), num_seq,
        _lib.ptr(kv_cache), kv_cache.stride(0), kv_cache.stride(1), kv_cache.stride(2), kv_cache.stride(3),
        total_tokens, num_heads, head_dim, int(page_size), _lib.stream_of(k),
    )
    _lib.check(rc, "update_kv_padded")


torch.library.define("mylib::update_kv", _SCHEMA)
torch.library.define("mylib::update_kv_padded", _SCHEMA)


@torch.library.impl("mylib::update_kv", "cuda")
def update_kv(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_last_page_len, page_size):
    paged_kv_append(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_last_page_len,
                    page_size)


@torch.library.impl("mylib::update_kv_padded", "cuda")
def update_kv_padded(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_last_page_len,
                     page_size):
    paged_kv_append(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_last_page_len,
                    page_size)


@torch.library.register_fake("mylib::update_kv")
def update_kv_abstract(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr, kv_last_page_len,
                       page_size):
    return None


@torch.library.register_fake("mylib::update_kv_padded")
def update_kv_padded_abstract(k, v, kv_append_indptr, kv_cache, kv_page_indices, kv_page_indptr,
                              kv_last_page_len, page_size):
    return None
