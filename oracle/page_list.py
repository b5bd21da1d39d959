"""Mixed draft/verify page-list build, restated on the CPU (test infrastructure only).

Follows ``aspire/models/sparse_draft_runner.py:126-153`` (``build_unified_indices``)
and the Triton copy kernel at ``sparse_draft_runner.py:92-123``, plus the
padding-row tail fill at ``aspire/backends/base.py:1253-1256``. DRAFT_MODE is 0
and VERIFY_MODE is 1 (``aspire/models/mixed_runner.py:9-10``).

The Triton kernel reads row ``b`` of the source table at flat offset
``b * width + i`` with a mask only on ``i < n_pages`` (no check against the row
width), so a count larger than the width continues into the next row; this
restatement reads the flattened table the same way.

Pinned by: the hand-worked known-answer case and the invariants in
``tests/test_oracle_page_list.py``; the kernel is compared to this bit-exactly.
"""

from __future__ import annotations

import numpy as np

DRAFT_MODE = 0
VERIFY_MODE = 1


def build_unified_indices(
    mode_flags: np.ndarray,
    draft_indices: np.ndarray,
    verify_indices: np.ndarray,
    draft_num_pages: np.ndarray,
    verify_num_pages: np.ndarray,
    paged_kv_indices: np.ndarray,
    paged_kv_indptr: np.ndarray,
) -> None:
    """Fill ``paged_kv_indptr[:B+1]`` and ``paged_kv_indices[:indptr[B]]`` in place."""
    bsz = mode_flags.shape[0]
    is_draft = np.asarray(mode_flags) == DRAFT_MODE
    n = np.where(is_draft, draft_num_pages, verify_num_pages).astype(np.int64)
    paged_kv_indptr[0] = 0
    paged_kv_indptr[1 : bsz + 1] = np.cumsum(n)
    d_flat = np.asarray(draft_indices).reshape(-1)
    v_flat = np.asarray(verify_indices).reshape(-1)
    d_width = draft_indices.shape[1]
    v_width = verify_indices.shape[1]
    for b in range(bsz):
        start = int(paged_kv_indptr[b])
        cnt = int(n[b])
        if cnt <= 0:
            continue
        if is_draft[b]:
            src = d_flat[b * d_width : b * d_width + cnt]
        else:
            src = v_flat[b * v_width : b * v_width + cnt]
        paged_kv_indices[start : start + cnt] = src


def fill_padding_rows(paged_kv_indptr: np.ndarray, last_page_len: np.ndarray, bsz: int) -> None:
    """base.py:1253-1256: padding rows repeat the final indptr and have no last page."""
    paged_kv_indptr[bsz + 1 :] = paged_kv_indptr[bsz]
    last_page_len[bsz:] = 0


def build_head_page_lists(mode_flags, selected, selected_counts, verify_indices, verify_num_pages,
                          paged_kv_indices: np.ndarray, paged_kv_indptr: np.ndarray,
                          share_verify: bool = False) -> None:
    """Per-(row, kv head) segments (no reference code: the consumer of the key-mean
    selection). Segment ``b*H + g`` is ``selected[b, g, :counts[b, g]]`` for a draft row
    and ``verify_indices[b, :verify_num_pages[b]]`` otherwise, written once per head or,
    with ``share_verify``, once per row. ``paged_kv_indptr[s]`` is segment ``s``'s first
    entry and ``paged_kv_indptr[B*H]`` the total. With one head and no sharing this is
    ``build_unified_indices`` above."""
    mode_flags = np.asarray(mode_flags)
    selected = np.asarray(selected)
    counts = np.asarray(selected_counts)
    bsz, heads = mode_flags.shape[0], selected.shape[1]
    pos = 0
    for b in range(bsz):
        row_start = pos
        for g in range(heads):
            if mode_flags[b] == DRAFT_MODE:
                paged_kv_indptr[b * heads + g] = pos
                src = selected[b, g, : int(counts[b, g])]
            elif share_verify:
                paged_kv_indptr[b * heads + g] = row_start
                if g > 0:
                    continue
                src = np.asarray(verify_indices)[b, : int(verify_num_pages[b])]
            else:
                paged_kv_indptr[b * heads + g] = pos
                src = np.asarray(verify_indices)[b, : int(verify_num_pages[b])]
            paged_kv_indices[pos : pos + len(src)] = src
            pos += len(src)
    paged_kv_indptr[bsz * heads] = pos
