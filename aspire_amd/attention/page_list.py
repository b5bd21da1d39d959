"""Mixed draft/verify page-list construction (HIP implementation).

Drop-in for ``build_unified_indices`` (``aspire/models/sparse_draft_runner.py:126-153``):
row ``b`` attends ``draft_num_pages[b]`` pages of ``draft_indices[b]`` when
``mode_flags[b] == DRAFT_MODE`` and ``verify_num_pages[b]`` pages of
``verify_indices[b]`` otherwise; ``paged_kv_indptr[:B+1]`` receives the running
page counts and ``paged_kv_indices`` the concatenated lists. The reference's
eager cumsum plus Triton copy become one kernel launch.
"""

from __future__ import annotations

import torch

from aspire_amd import _lib

DRAFT_MODE = 0
VERIFY_MODE = 1


def build_unified_indices(
    mode_flags: torch.Tensor,
    draft_indices: torch.Tensor,
    verify_indices: torch.Tensor,
    draft_num_pages: torch.Tensor,
    verify_num_pages: torch.Tensor,
    paged_kv_indices: torch.Tensor,
    paged_kv_indptr: torch.Tensor,
    *,
    indptr_fill_to: int | None = None,
) -> None:
    """Fill ``paged_kv_indptr`` / ``paged_kv_indices`` in place.

    ``indptr_fill_to`` (not in the reference signature) additionally repeats
    ``indptr[B]`` up to that length, the padding-row fill the reference does
    right after this call (aspire/backends/base.py:1253-1255).
    """
    batch = mode_flags.shape[0]
    _lib.require_cuda(mode_flags, paged_kv_indices, paged_kv_indptr, what="build_unified_indices")
    for name, t in (("draft_indices", draft_indices), ("verify_indices", verify_indices),
                    ("draft_num_pages", draft_num_pages), ("verify_num_pages", verify_num_pages),
                    ("paged_kv_indices", paged_kv_indices), ("paged_kv_indptr", paged_kv_indptr)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"build_unified_indices: {name} must be a contiguous int32 tensor")
    if mode_flags.dtype == torch.bool:
        flags, esize = mode_flags.view(torch.uint8), 1
    elif mode_flags.element_size() in (1, 4, 8) and not mode_flags.is_floating_point():
        flags, esize = mode_flags, mode_flags.element_size()
    else:
        raise ValueError("build_unified_indices: mode_flags must be an integer or bool tensor")
    flags = flags.contiguous()
    fill = batch + 1 if indptr_fill_to is None else int(indptr_fill_to)
    if fill > paged_kv_indptr.shape[0]:
        raise ValueError("build_unified_indices: indptr_fill_to exceeds paged_kv_indptr")
    if paged_kv_indptr.shape[0] < batch + 1:
        raise ValueError("build_unified_indices: paged_kv_indptr needs batch + 1 entries")
    d_rows = draft_indices.shape[0] if draft_indices.dim() > 1 else 1
    v_rows = verify_indices.shape[0] if verify_indices.dim() > 1 else 1
    rc = _lib.lib().aspire_build_mixed_page_list(
        _lib.ptr(flags), esize,
        _lib.ptr(draft_indices), draft_indices.shape[-1], d_rows,
        _lib.ptr(verify_indices), verify_indices.shape[-1], v_rows,
        _lib.ptr(draft_num_pages), _lib.ptr(verify_num_pages), batch,
        _lib.ptr(paged_kv_indices), paged_kv_indices.numel(),
        _lib.ptr(paged_kv_indptr), fill, _lib.stream_of(paged_kv_indptr),
    )
    _lib.check(rc, "build_unified_indices")


def build_head_page_lists(
    mode_flags: torch.Tensor,
    selected: torch.Tensor,
    selected_counts: torch.Tensor,
    verify_indices: torch.Tensor,
    verify_num_pages: torch.Tensor,
    paged_kv_indices: torch.Tensor,
    paged_kv_indptr: torch.Tensor,
    *,
    share_verify: bool = False,
    indptr_fill_to: int | None = None,
) -> None:
    """Per-(row, kv head) lists for a plan made with ``per_head_lists=True`` (or,
    with ``share_verify``, for ``plan_segments``).

    Not in the reference: this consumes the key-mean selection
    (``KeyMeanPageSelector.select``: ``selected [B, H_kv, k]``, ``selected_counts
    [B, H_kv]``). Segment ``b * H_kv + g`` lists ``selected[b, g, :count]`` when
    row ``b`` drafts and ``verify_indices[b, :verify_num_pages[b]]`` otherwise,
    once per head or, with ``share_verify``, once per row for all its heads.
    ``paged_kv_indptr[s]`` receives segment ``s``'s first entry and
    ``paged_kv_indptr[B * H_kv]`` the total (the running counts without sharing).
    """
    batch = mode_flags.shape[0]
    if selected.dim() != 3 or selected.shape[0] < batch or selected_counts.shape[:2] != selected.shape[:2]:
        raise ValueError("build_head_page_lists: selected must be [B, H_kv, k] with counts [B, H_kv]")
    heads = selected.shape[1]
    _lib.require_cuda(mode_flags, selected, selected_counts, verify_indices, verify_num_pages, paged_kv_indices,
                      paged_kv_indptr, what="build_head_page_lists")
    for name, t in (("selected", selected), ("selected_counts", selected_counts), ("verify_indices", verify_indices),
                    ("verify_num_pages", verify_num_pages), ("paged_kv_indices", paged_kv_indices),
                    ("paged_kv_indptr", paged_kv_indptr)):
        if t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"build_head_page_lists: {name} must be a contiguous int32 tensor")
    if mode_flags.dtype == torch.bool:
        flags, esize = mode_flags.view(torch.uint8), 1
    elif mode_flags.element_size() in (1, 4, 8) and not mode_flags.is_floating_point():
        flags, esize = mode_flags, mode_flags.element_size()
    else:
        raise ValueError("build_head_page_lists: mode_flags must be an integer or bool tensor")
    flags = flags.contiguous()
    segs = batch * heads
    fill = segs + 1 if indptr_fill_to is None else int(indptr_fill_to)
    if paged_kv_indptr.shape[0] < max(fill, segs + 1):
        raise ValueError("build_head_page_lists: paged_kv_indptr needs B * H_kv + 1 entries (and the fill)")
    v_rows = verify_indices.shape[0] if verify_indices.dim() > 1 else 1
    rc = _lib.lib().aspire_build_head_page_lists(
        _lib.ptr(flags), esize, _lib.ptr(selected), selected.shape[-1], _lib.ptr(selected_counts),
        _lib.ptr(verify_indices), verify_indices.shape[-1], v_rows, _lib.ptr(verify_num_pages), batch, heads,
        1 if share_verify else 0, _lib.ptr(paged_kv_indices), paged_kv_indices.numel(), _lib.ptr(paged_kv_indptr), fill,
        _lib.stream_of(paged_kv_indptr),
    )
    _lib.check(rc, "build_head_page_lists")
