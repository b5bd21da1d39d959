"""Paged KV append, restated on the CPU (test infrastructure only).

Follows ``aspire/attention/kv_ops.py:127-187`` (``update_kv_padded``) and the
Triton kernel it launches, ``kv_ops.py:63-124``. Two helpers come from the
un-vendored FlashInfer dependency pinned at commit
``56ed54098411946525da17eca2bcfd7ec72a515e`` (scripts/install_flashinfer.sh:4-5):

* ``flashinfer.get_seq_lens(indptr, last_page_len, page_size)``: per row,
  ``clamp(indptr[b+1] - indptr[b] - 1, 0) * page_size + last_page_len[b]``.
  The reference restates the same formula at
  ``aspire/backends/host_plan.py:243-246`` and ``aspire/backends/base.py:929-933``.
* ``flashinfer.triton.page.get_batch_indices_positions_kernel``: launched with
  one program per entry of ``seq_lens`` (kv_ops.py:148-156); for row ``b`` and
  token ``i`` in ``[append_indptr[b], append_indptr[b+1])`` it writes
  ``batch = b`` and ``pos = i + seq_lens[b] - append_indptr[b+1]``. Tokens no row
  covers keep the defaults set at kv_ops.py:144-147 (batch 0, position -1).

Pinned by: the hand-worked known-answer case and the round-trip/untouched-bytes
invariants in ``tests/test_oracle_append.py``; the kernel is compared to this
bit-exactly.
"""

from __future__ import annotations

import numpy as np


def seq_lens(kv_page_indptr: np.ndarray, kv_last_page_len: np.ndarray, page_size: int) -> np.ndarray:
    """``get_seq_lens``: one entry per ``kv_last_page_len`` row."""
    indptr = np.asarray(kv_page_indptr, dtype=np.int64)
    last = np.asarray(kv_last_page_len, dtype=np.int64)
    n = last.shape[0]
    pages = indptr[1 : n + 1] - indptr[:n]
    return np.maximum(pages - 1, 0) * page_size + last


def batch_indices_positions(append_indptr: np.ndarray, lens: np.ndarray, total_tokens: int):
    """``get_batch_indices_positions``: (batch index, position) per appended token."""
    indptr = np.asarray(append_indptr, dtype=np.int64)
    batch = np.zeros(total_tokens, dtype=np.int64)
    pos = np.full(total_tokens, -1, dtype=np.int64)
    for b in range(lens.shape[0]):
        start, end = int(indptr[b]), int(indptr[b + 1])
        for i in range(max(start, 0), min(end, total_tokens)):
            batch[i] = b
            pos[i] = i + int(lens[b]) - end
    return batch, pos


def paged_kv_append(
    k: np.ndarray,
    v: np.ndarray,
    append_indptr: np.ndarray,
    cache: np.ndarray,
    kv_indices: np.ndarray,
    kv_indptr: np.ndarray,
    last_page_len: np.ndarray,
    page_size: int,
    *,
    inplace: bool = False,
) -> np.ndarray:
    """Return a copy of ``cache`` with the new K/V rows scattered in (``inplace``:
    scatter into ``cache`` itself and return it, as the reference mutates its cache).

    ``k``/``v``: ``[T, H_kv, D]`` (any dtype; bf16 is passed as its uint16
    bits); ``cache``: ``[P, 2, page_size, H_kv, D]`` of the same dtype. The skip
    rules are kv_ops.py:92-98 and the page/slot arithmetic kv_ops.py:100-103.
    """
    out = cache if inplace else cache.copy()
    total = k.shape[0]
    if total == 0:
        return out
    lens = seq_lens(kv_indptr, last_page_len, page_size)
    batch, pos = batch_indices_positions(append_indptr, lens, total)
    indptr = np.asarray(kv_indptr, dtype=np.int64)
    last = np.asarray(last_page_len, dtype=np.int64)
    for i in range(total):
        b, p = int(batch[i]), int(pos[i])
        if p < 0:
            continue
        start, end = int(indptr[b]), int(indptr[b + 1])
        count = end - start
        if count == 0:
            continue
        length = (count - 1) * page_size + int(last[b])
        if p >= length:
            continue
        abs_pos = start * page_size + p
        page_iter = abs_pos // page_size
        entry = abs_pos - page_iter * page_size
        phys = int(kv_indices[page_iter])
        out[phys, 0, entry] = k[i]
        out[phys, 1, entry] = v[i]
    return out
