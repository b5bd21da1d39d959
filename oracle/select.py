"""Page scoring and top-k page selection, restated on the CPU (test infrastructure only).

(R) The reference selector ``PageSelectorFirstLastAvg.select``
    (``aspire/backends/page_selector.py:206-214``) ->
    ``_select_first_last_impl`` (163-181) -> ``_finalize_scores`` (79-108), with
    ``compute_valid_counts`` (52-62) and ``_view_buffer`` (132-138). Restated
    with the same torch ops in the same order, so the fp16 rounding of
    ``logits * sm_scale*log2(e)`` (page_selector.py:170), the
    ``nan_to_num_(nan=-inf)`` defaults, the ``-j*1e-7`` position bias and the
    sentinel sort reproduce.
    Pinned by the golden vectors in ``tests/golden/select_first_last.npz``,
    written by ``tests/golden/make_select_golden.py`` from the reference's own
    ``page_selector.py`` (loaded by file path in the build container), plus the
    one-hot and all-pages special cases in ``tests/test_oracle_select.py``.

    Ordering: the reference sorts a row's selected pages by *physical* page id
    (page_selector.py:102-106). Draft appends write into the tail entry of the
    list (base.py:1207-1213, kv_ops.py:96-103), which is only the current page
    when the block table is increasing (the reference's table is an arange,
    sparse_draft_runner.py:248-250). ``order="logical"`` sorts by logical page
    index instead and gives the identical result for an increasing table;
    ``order="physical"`` is the reference's literal rule.

(B) The per-(request, KV head) key-mean selector of BASELINE config 2, which
    has no reference counterpart: page ``j`` of kv head ``g`` scores
    ``max_{h in group(g)} q_h . mean_t(k_{j,t,g})`` (``oracle.attention``'s
    page-score epilogue); the top ``k`` pages per (request, kv head) are kept,
    optionally forcing the last ``L`` pages, and listed in ascending logical
    order. Pinned by a brute-force loop on tiny inputs in
    ``tests/test_oracle_select.py``.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F


class FirstLastSelector:
    """CPU twin of ``PageSelectorFirstLastAvg`` (constructor arguments of page_selector.py:9-12)."""

    def __init__(
        self,
        *,
        pages_per_slot: int,
        subset_cache_size: int,
        L: int,
        n_heads: int,
        page_size: int,
        max_seq_length: int,
        bsz: int,
        head_dim: int = 128,
        kv_stride: int | None = None,
        draft_percent: float | None = None,
        min_draft_pages: int | None = None,
    ):
        self.subset_cache_size = subset_cache_size
        self.L = L
        self._min_draft_pages = min_draft_pages
        self.n_heads = n_heads
        self.page_size = page_size
        self.max_seq_length = max_seq_length
        self._kv_stride = kv_stride or max_seq_length
        self.pages_per_slot = pages_per_slot
        self._draft_percent = draft_percent
        self._bsz = bsz
        sm_scale = 1.0 / math.sqrt(head_dim)
        self._sm_scale_log2e = sm_scale * math.log2(math.e)
        self._seq_pad = pages_per_slot * page_size - max_seq_length
        self._j = torch.arange(pages_per_slot)
        self._pos_bias = -torch.arange(pages_per_slot, dtype=torch.float32) * 1e-7
        self._col_ids = torch.arange(subset_cache_size, dtype=torch.int32)
        self._sentinel = torch.iinfo(torch.int32).max

    def compute_valid_counts(self, num_pages: torch.Tensor) -> torch.Tensor:
        """page_selector.py:52-62."""
        hi = num_pages.clamp(max=self.subset_cache_size).to(torch.int32)
        if self._draft_percent is None:
            if self._min_draft_pages is not None:
                return num_pages.clamp(max=self._min_draft_pages).to(torch.int32)
            return hi
        floor = self._min_draft_pages if self._min_draft_pages is not None else self.L
        lo = num_pages.clamp(max=floor).to(torch.int32)
        target = (num_pages.float() * self._draft_percent / 100).ceil_().to(torch.int32)
        return torch.clamp(target, lo, hi)

    def page_scores(self, dump_flat, lse_buffer, qo_indptr) -> torch.Tensor:
        """Pre-finalize page scores ``[B, pages_per_slot]`` (page_selector.py:168-180)."""
        B = self._bsz
        logits = dump_flat.view(B, self.n_heads, 2, self._kv_stride)
        if self._kv_stride != self.max_seq_length:
            logits = logits[..., : self.max_seq_length]
        max_q_idx = max(lse_buffer.shape[0] - 1, 0)
        first_q = qo_indptr[:B].long().clamp(min=0, max=max_q_idx)
        last_q = (qo_indptr[1 : B + 1].long() - 1).clamp(min=0, max=max_q_idx)
        lse = torch.stack([lse_buffer[first_q], lse_buffer[last_q]], dim=2)
        norm = logits * self._sm_scale_log2e - lse[:, :, :, None]
        norm.nan_to_num_(nan=float("-inf"))
        token_scores = torch.exp2(norm).amax(dim=1).sum(dim=1)
        if self._seq_pad > 0:
            token_scores = F.pad(token_scores, (0, self._seq_pad))
        scores = token_scores.view(B, self.pages_per_slot, self.page_size).sum(dim=-1)
        scores.add_(self._pos_bias)
        return scores

    def finalize(self, scores, num_pages, block_table, order: str = "physical"):
        """page_selector.py:79-108 (``order="logical"`` sorts before the gather)."""
        scores = scores.clone()
        np_long = num_pages.long()
        j = self._j[None]
        last_start = (np_long - self.L).clamp_(min=0)
        last_mask = (j >= last_start[:, None]) & (j < np_long[:, None])
        scores[last_mask] = float("inf")
        scores[j >= np_long[:, None]] = float("-inf")
        _, topk_idx = scores.topk(self.subset_cache_size, dim=1)
        topk_idx.clamp_(max=block_table.shape[1] - 1)
        valid = self.compute_valid_counts(num_pages)
        valid_mask = self._col_ids[None, :] < valid[:, None]
        if order == "physical":
            selected = torch.gather(block_table.to(torch.int32), 1, topk_idx)
            selected[~valid_mask] = self._sentinel
            selected, _ = selected.sort(dim=1)
            selected[~valid_mask] = 0
        elif order == "logical":
            logical = topk_idx.to(torch.int32)
            logical[~valid_mask] = self._sentinel
            logical, _ = logical.sort(dim=1)
            logical[~valid_mask] = 0
            selected = torch.gather(block_table.to(torch.int32), 1, logical.long())
            selected[~valid_mask] = 0
        else:
            raise ValueError(f"unknown order {order!r}")
        return selected, valid

    def select(self, dump_flat, lse_buffer, num_pages, block_table, qo_indptr, order: str = "physical"):
        scores = self.page_scores(dump_flat, lse_buffer, qo_indptr)
        return self.finalize(scores, num_pages, block_table, order=order)

    def effective_scores(self, scores, num_pages) -> torch.Tensor:
        """Scores after the last-L / out-of-range forcing (for gap-aware set checks)."""
        scores = scores.clone()
        np_long = num_pages.long()
        j = self._j[None]
        last_start = (np_long - self.L).clamp_(min=0)
        scores[(j >= last_start[:, None]) & (j < np_long[:, None])] = float("inf")
        scores[j >= np_long[:, None]] = float("-inf")
        return scores


def topk_pages_per_head(scores: torch.Tensor, num_pages, k: int, L: int = 0):
    """(B) selection: ``scores [S, max_pages]`` for S = B*H_kv segments with
    ``num_pages[s]`` valid pages each. Returns ``(logical [S, k] int32, counts [S])``:
    the top ``min(k, num_pages)`` pages in ascending logical order, zero-padded,
    with the last ``L`` pages of each segment forced in."""
    S, width = scores.shape
    out = torch.zeros((S, k), dtype=torch.int32)
    counts = torch.zeros(S, dtype=torch.int32)
    for s in range(S):
        n = int(num_pages[s])
        take = min(k, n)
        counts[s] = take
        if take == 0:
            continue
        sc = scores[s, :n].clone()
        if L > 0:
            sc[max(n - L, 0) : n] = float("inf")
        idx = torch.topk(sc, take).indices.sort().values
        out[s, :take] = idx.to(torch.int32)
    return out, counts
