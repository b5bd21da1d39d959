"""Page selection after the refresh-layer dump (HIP implementation).

Drop-in for ``aspire/backends/page_selector.py``: ``PageSelector`` (last-token
dump, page_selector.py:7-157) and ``PageSelectorFirstLastAvg`` (first/last
dump, page_selector.py:160-233) keep their constructor, ``compute_valid_counts``,
``select`` and ``select_subset``. Each select is two launches of
libaspire_hip.so: ``aspire_select_first_last_scores`` (the element-wise
normalise/exp2/max-over-heads/sum-over-slots chain and the per-page sums, over
pages below each row's count only) and ``aspire_select_topk`` (forced last-L
pages, radix top-k, block-table lookup, sort). Outputs land in preallocated
buffers, so a select is graph-capturable like the reference's.

Ordering: the reference sorts each row's pages by physical id
(page_selector.py:102-106); the draft KV append writes into the tail entry of
the list (base.py:1207-1213), which is the current page only when the block
table increases along the row (the reference's table is an arange,
sparse_draft_runner.py:248-250). ``order="logical"`` (default) sorts by logical
page index, identical to the reference for an increasing table and correct for
any table; ``order="physical"`` reproduces the reference's rule literally.

``KeyMeanPageSelector`` is the per-(request, KV head) selector of BASELINE
config 2, which has no reference counterpart: page scores come from the
attention kernel's key-mean epilogue (``HolisticAttentionWrapper.run(...,
page_scores=...)``) and the top ``k`` pages per (request, kv head) are kept.
"""

from __future__ import annotations

import math

import torch

from aspire_amd import _lib

_ORDERS = {"physical": 0, "logical": 1}


class PageSelector:
    """Selector over a one-slot (last verify token) logits dump."""

    _slots = 1

    def __init__(self, max_batch_size, pages_per_slot, subset_cache_size, L, n_heads, page_size,
                 max_seq_length, device, bsz, dec_len, head_dim=128, kv_stride=None, draft_percent=None,
                 min_draft_pages=None, order: str = "logical"):
        if order not in _ORDERS:
            raise ValueError(f"order must be one of {sorted(_ORDERS)}")
        self.subset_cache_size = subset_cache_size
        self.L = L
        self._min_draft_pages = min_draft_pages
        self.n_heads = n_heads
        self.page_size = page_size
        self.max_seq_length = max_seq_length
        self._kv_stride = kv_stride or max_seq_length
        self.pages_per_slot = pages_per_slot
        self.device = torch.device(device)
        self._draft_percent = draft_percent
        self._bsz = bsz
        self._dec_len = dec_len
        self._order = order
        sm_scale = 1.0 / math.sqrt(head_dim)
        self._sm_scale_log2e = sm_scale * math.log2(math.e)
        self._max_finalize_B = max_batch_size
        self._scores = torch.empty(max_batch_size, pages_per_slot, dtype=torch.float32, device=self.device)
        k = subset_cache_size
        self._selected_buf = torch.empty(max_batch_size, max(k, 1), dtype=torch.int32, device=self.device)
        self._valid_counts_buf = torch.empty(max_batch_size, dtype=torch.int32, device=self.device)
        self._sentinel = torch.iinfo(torch.int32).max

    def compute_valid_counts(self, num_pages: torch.Tensor) -> torch.Tensor:
        """Per-request draft page count (page_selector.py:52-62), in torch."""
        hi = num_pages.clamp(max=self.subset_cache_size).to(torch.int32)
        if self._draft_percent is None:
            if self._min_draft_pages is not None:
                return num_pages.clamp(max=self._min_draft_pages).to(torch.int32)
            return hi
        floor = self._min_draft_pages if self._min_draft_pages is not None else self.L
        lo = num_pages.clamp(max=floor).to(torch.int32)
        target = (num_pages.float() * self._draft_percent / 100).ceil_().to(torch.int32)
        return torch.clamp(target, lo, hi)

    def _count_mode(self):
        if self._draft_percent is None:
            if self._min_draft_pages is not None:
                return 1, self.subset_cache_size, int(self._min_draft_pages), 0.0
            return 0, self.subset_cache_size, 0, 0.0
        floor = self._min_draft_pages if self._min_draft_pages is not None else self.L
        return 2, self.subset_cache_size, int(floor), float(self._draft_percent)

    def _buffers(self, rows):
        if rows <= self._max_finalize_B:
            return self._scores[:rows], self._selected_buf[:rows], self._valid_counts_buf[:rows]
        return (torch.empty(rows, self.pages_per_slot, dtype=torch.float32, device=self.device),
                torch.empty(rows, max(self.subset_cache_size, 1), dtype=torch.int32, device=self.device),
                torch.empty(rows, dtype=torch.int32, device=self.device))

    def _run(self, attention_weights_buffer, lse_buffer, num_pages, block_table, qo_indptr, row_ids, rows):
        _lib.require_cuda(attention_weights_buffer, lse_buffer, num_pages, block_table, qo_indptr,
                          what="PageSelector.select")
        if attention_weights_buffer.dtype != torch.float16:
            raise ValueError("the HIP selector reads an fp16 logits dump")
        need = self._bsz * self.n_heads * self._slots * self._kv_stride
        if attention_weights_buffer.numel() < need:
            raise ValueError(f"dump buffer holds {attention_weights_buffer.numel()} elements, need {need}")
        for name, t in (("num_pages", num_pages), ("block_table", block_table), ("qo_indptr", qo_indptr)):
            if t.dtype != torch.int32:
                raise ValueError(f"PageSelector: {name} must be int32")
        lse = lse_buffer.contiguous()
        if lse.dtype != torch.float32 or lse.dim() != 2 or lse.shape[1] != self.n_heads:
            raise ValueError("lse_buffer must be fp32 [rows, n_heads]")
        qo = qo_indptr.contiguous()
        npg = num_pages.contiguous()
        if qo.numel() < self._bsz + 1 or npg.numel() < self._bsz or block_table.shape[0] < self._bsz:
            raise ValueError("qo_indptr, num_pages and block_table must cover bsz rows")
        if block_table.stride(1) != 1:
            raise ValueError("block_table rows must be contiguous")
        scores, selected, valid = self._buffers(rows)
        stream = _lib.stream_of(attention_weights_buffer)
        L = _lib.lib()
        rc = L.aspire_select_first_last_scores(
            _lib.ptr(attention_weights_buffer), self._kv_stride, self.n_heads, self._bsz, self.max_seq_length,
            _lib.ptr(lse), lse.shape[0], _lib.ptr(qo), _lib.ptr(npg), _lib.ptr(row_ids), rows, self.page_size,
            float(self._sm_scale_log2e), _lib.ptr(scores), scores.stride(0), self._slots, stream)
        _lib.check(rc, "PageSelector.select")
        mode, subset, min_pages, pct = self._count_mode()
        rc = L.aspire_select_topk(
            _lib.ptr(scores), scores.stride(0), _lib.ptr(npg), _lib.ptr(row_ids), rows, 1, int(self.L), mode,
            int(subset), int(min_pages), float(pct), _lib.ptr(block_table), block_table.stride(0),
            _ORDERS[self._order], _lib.ptr(selected), selected.stride(0), self.subset_cache_size,
            _lib.ptr(valid), stream)
        _lib.check(rc, "PageSelector.select")
        return selected[:, : self.subset_cache_size], valid

    def select(self, attention_weights_buffer, lse_buffer, num_pages, block_table, qo_indptr):
        return self._run(attention_weights_buffer, lse_buffer, num_pages, block_table, qo_indptr, None,
                         self._bsz)

    def select_subset(self, slot_ids, attention_weights_buffer, lse_buffer, num_pages, block_table, qo_indptr):
        if slot_ids.numel() == 0:
            empty = block_table.new_empty((0, self.subset_cache_size), dtype=torch.int32)
            return empty, torch.zeros(0, dtype=torch.int32, device=self.device)
        rows = slot_ids.to(device=self.device, dtype=torch.int32).contiguous()
        return self._run(attention_weights_buffer, lse_buffer, num_pages, block_table, qo_indptr, rows,
                         rows.numel())


class PageSelectorFirstLastAvg(PageSelector):
    """Selector over the compact first/last verify-token dump (two slots per head)."""

    _slots = 2

    def _run_compact(self, logits, first_lse, last_lse, num_pages, block_table):
        """Scores + top-k over ``logits [R, H, 2, S]`` with per-row LSEs ``[R, H]``: the LSE rows
        are stacked as (first, last) pairs and addressed through qo_indptr = [0, 2, ..., 2R],
        so the kernels read exactly the rows select() reads through the token indptr."""
        R, H = logits.shape[0], logits.shape[1]
        if logits.dim() != 4 or logits.shape[2] != 2 or H != self.n_heads:
            raise ValueError("logits must be [rows, n_heads, 2, seq_len]")
        if first_lse.shape != (R, H) or last_lse.shape != (R, H):
            raise ValueError("first_lse and last_lse must be [rows, n_heads]")
        if logits.dtype != torch.float16:
            raise ValueError("the HIP selector reads an fp16 logits dump")
        stride = logits.stride(2)
        if logits.stride(3) != 1 or logits.stride(1) != 2 * stride or logits.stride(0) != H * 2 * stride:
            logits = logits.contiguous()
            stride = logits.shape[3]
        seq_len = logits.shape[3]
        if seq_len > self.pages_per_slot * self.page_size:
            raise ValueError("seq_len exceeds pages_per_slot * page_size")
        if num_pages.dtype != torch.int32 or block_table.dtype != torch.int32 or block_table.stride(1) != 1:
            raise ValueError("num_pages and block_table must be int32 with contiguous rows")
        if num_pages.numel() < R or block_table.shape[0] < R:
            raise ValueError("num_pages and block_table must cover every row")
        _lib.require_cuda(logits, first_lse, last_lse, num_pages, block_table,
                          what="PageSelectorFirstLastAvg.select_from_compact_first_last")
        lse = torch.stack([first_lse, last_lse], dim=1).to(torch.float32).reshape(2 * R, H).contiguous()
        qo = torch.arange(0, 2 * R + 1, 2, dtype=torch.int32, device=logits.device)
        npg = num_pages.contiguous()
        scores, selected, valid = self._buffers(R)
        stream = _lib.stream_of(logits)
        L = _lib.lib()
        rc = L.aspire_select_first_last_scores(
            _lib.ptr(logits), stride, self.n_heads, R, seq_len, _lib.ptr(lse), 2 * R, _lib.ptr(qo), _lib.ptr(npg),
            None, R, self.page_size, float(self._sm_scale_log2e), _lib.ptr(scores), scores.stride(0), 2, stream)
        _lib.check(rc, "PageSelectorFirstLastAvg.select_from_compact_first_last")
        mode, subset, min_pages, pct = self._count_mode()
        rc = L.aspire_select_topk(
            _lib.ptr(scores), scores.stride(0), _lib.ptr(npg), None, R, 1, int(self.L), mode, int(subset),
            int(min_pages), float(pct), _lib.ptr(block_table), block_table.stride(0), _ORDERS[self._order],
            _lib.ptr(selected), selected.stride(0), self.subset_cache_size, _lib.ptr(valid), stream)
        _lib.check(rc, "PageSelectorFirstLastAvg.select_from_compact_first_last")
        return selected[:, : self.subset_cache_size], valid

    def select_from_compact_first_last(self, logits, first_lse, last_lse, num_pages, block_table):
        """``logits [B, H, 2, seq_len]`` (a view of the dump is fine), ``first_lse`` / ``last_lse``
        ``[B, H]``: the same selection as ``select`` with the LSEs given per row
        (page_selector.py:183-184)."""
        return self._run_compact(logits, first_lse, last_lse, num_pages, block_table)

    def select_layers_from_compact_first_last(self, logits, first_lse, last_lse, num_pages, block_table):
        """``logits [n_layers, B, H, 2, kv_stride]``, LSEs ``[n_layers, B, H]``: every layer's rows
        selected in one pass (page counts and tables repeated per layer); returns
        ``(selected [n_layers, B, k], valid_counts [B])`` (page_selector.py:186-204)."""
        n_layers, batch = logits.shape[:2]
        flat = logits.reshape(n_layers * batch, self.n_heads, 2, logits.shape[-1])
        if flat.shape[-1] != self.max_seq_length:
            flat = flat[..., : self.max_seq_length]
        selected, valid = self._run_compact(
            flat, first_lse.reshape(n_layers * batch, self.n_heads), last_lse.reshape(n_layers * batch, self.n_heads),
            num_pages[:batch].to(torch.int32).repeat(n_layers).contiguous(),
            block_table[:batch].repeat(n_layers, 1).contiguous())
        return selected.view(n_layers, batch, self.subset_cache_size), valid[:batch]


class KeyMeanPageSelector:
    """Top-k pages per (request, KV head) by the key-mean score.

    ``page_scores`` is the ``[max_batch * H_kv, max_pages]`` fp32 buffer to pass
    to ``HolisticAttentionWrapper.run(..., page_scores=...)``; ``select`` then
    keeps ``min(k, num_pages)`` pages per (request, kv head), with the last
    ``L`` pages forced in, as physical ids in ascending logical order.
    """

    def __init__(self, max_batch_size: int, num_kv_heads: int, max_pages: int, k: int, L: int = 0,
                 device="cuda", order: str = "logical"):
        if order not in _ORDERS:
            raise ValueError(f"order must be one of {sorted(_ORDERS)}")
        self.num_kv_heads = num_kv_heads
        self.k = k
        self.L = L
        self.max_pages = max_pages
        self._order = order
        self.device = torch.device(device)
        self.page_scores = torch.empty(max_batch_size * num_kv_heads, max_pages, dtype=torch.float32,
                                       device=self.device)
        self.selected = torch.zeros(max_batch_size, num_kv_heads, k, dtype=torch.int32, device=self.device)
        self.counts = torch.zeros(max_batch_size, num_kv_heads, dtype=torch.int32, device=self.device)

    def select(self, num_pages: torch.Tensor, block_table: torch.Tensor, batch: int | None = None):
        batch = num_pages.shape[0] if batch is None else batch
        _lib.require_cuda(num_pages, block_table, what="KeyMeanPageSelector.select")
        if num_pages.dtype != torch.int32 or block_table.dtype != torch.int32 or block_table.stride(1) != 1:
            raise ValueError("num_pages and block_table must be int32 with contiguous rows")
        if batch > self.selected.shape[0] or num_pages.numel() < batch or block_table.shape[0] < batch:
            raise ValueError("batch exceeds the selector's capacity or the num_pages / block_table rows")
        segs = batch * self.num_kv_heads
        rc = _lib.lib().aspire_select_topk(
            _lib.ptr(self.page_scores), self.page_scores.stride(0), _lib.ptr(num_pages.contiguous()), None,
            segs, self.num_kv_heads, int(self.L), 0, int(self.k), 0, 0.0, _lib.ptr(block_table),
            block_table.stride(0), _ORDERS[self._order], _lib.ptr(self.selected), self.k, self.k,
            _lib.ptr(self.counts), _lib.stream_of(num_pages))
        _lib.check(rc, "KeyMeanPageSelector.select")
        return self.selected[:batch], self.counts[:batch]
