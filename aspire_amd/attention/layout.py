"""Layout owners of the paged-KV path: the unified cache, page math, block table, buckets.

Same names and contracts as the reference's definitions, so callers of the
attention path find them here:

* ``KVCache`` — one ``[pages, 2, page_size, H_kv, head_dim]`` buffer holding
  target pages then draft pages, with ``kv_cache`` / ``draft_cache`` views and
  ``unified_cache`` (aspire/models/mixed_transformer.py:22-53). K is ``[:, 0]``,
  V is ``[:, 1]``; within a page the layout is NHD, the layout every kernel of
  this package reads.
* ``get_num_pages`` / ``get_last_page_len`` — the page math of
  ``_get_num_pages`` / ``_get_last_page_len`` (aspire/models/mixed_runner.py:98-120).
* ``static_block_table`` — the arange table and pages per request of the
  sparse-draft runner (aspire/models/sparse_draft_runner.py:240-250).
* ``graph_buckets`` / ``select_bucket`` — the CUDA-graph token buckets
  (aspire/engine/buffers.py:7-24).
* ``DRAFT_MODE`` / ``VERIFY_MODE`` (aspire/models/mixed_runner.py:9-10).
"""

from __future__ import annotations

import torch
from torch import nn

from aspire_amd.attention.page_list import DRAFT_MODE, VERIFY_MODE


def _mark_static(t: torch.Tensor) -> None:
    try:
        import torch._dynamo as dynamo

        dynamo.mark_static_address(t)
    except (ImportError, AttributeError, RuntimeError):
        pass


class KVCache(nn.Module):
    """The paged cache of one layer. With ``spec`` a single allocation holds the target
    pages followed by the draft pages, and ``kv_cache`` / ``draft_cache`` slice it
    (no second buffer); otherwise ``kv_cache`` is the whole allocation."""

    def __init__(self, max_num_pages: int, page_size: int, n_heads: int, head_dim: int,
                 dtype: torch.dtype = torch.bfloat16, spec: bool = False, draft_max_num_pages: int = 0,
                 device=None):
        super().__init__()
        self.page_size = page_size
        self.max_num_pages = max_num_pages
        self.draft_max_num_pages = draft_max_num_pages
        self.is_spec = spec
        pages = max_num_pages + (draft_max_num_pages if spec else 0)
        buf = torch.zeros((pages, 2, page_size, n_heads, head_dim), dtype=dtype, device=device)
        if spec:
            # [target pages 0 .. max_num_pages-1][draft pages max_num_pages .. end]
            self.register_buffer("_unified_kv_cache", buf)
            self.kv_cache = self._unified_kv_cache[:max_num_pages]
            self.draft_cache = self._unified_kv_cache[max_num_pages:]
            for t in (self._unified_kv_cache, self.kv_cache, self.draft_cache):
                _mark_static(t)
        else:
            self.register_buffer("kv_cache", buf)
            _mark_static(self.kv_cache)

    @property
    def unified_cache(self) -> torch.Tensor:
        """The whole buffer (target + draft pages): a view, never a copy."""
        return self._unified_kv_cache if self.is_spec else self.kv_cache


def get_num_pages(seq_lens: torch.Tensor, page_size: int) -> torch.Tensor:
    """Pages holding ``seq_lens`` tokens: ceil(len / page_size)."""
    return (seq_lens + page_size - 1) // page_size


def get_last_page_len(seq_lens: torch.Tensor, page_size: int) -> torch.Tensor:
    """Tokens in the last page: (len - 1) % page_size + 1, and 0 for an empty row."""
    return torch.where(seq_lens > 0, (seq_lens - 1) % page_size + 1, torch.zeros_like(seq_lens))


def static_block_table(max_batch_size: int, max_seq_length: int, page_size: int, device=None):
    """``(block_table [B, pages_per_request] int32, pages_per_request, max_num_pages)``: request b owns
    pages b * pages_per_request .. (b + 1) * pages_per_request - 1; a length that is not a whole
    number of pages gets one more page per request."""
    max_num_pages = max_batch_size * (max_seq_length // page_size)
    if max_num_pages * page_size < max_batch_size * max_seq_length:
        max_num_pages += max_batch_size
    per_request = max_num_pages // max_batch_size
    table = torch.arange(max_num_pages, dtype=torch.int32, device=device).reshape(max_batch_size, per_request)
    return table, per_request, max_num_pages


def graph_buckets(max_tokens: int) -> tuple[int, ...]:
    """Token counts graphs are captured for: 1, 2, 4, then every multiple of 8, and max_tokens."""
    if max_tokens < 1:
        raise ValueError(f"graph_buckets needs at least one token, got max_tokens={max_tokens}")
    sizes = {s for s in (1, 2, 4) if s <= max_tokens}
    sizes.update(range(8, max_tokens + 1, 8))
    sizes.add(max_tokens)
    return tuple(sorted(sizes))


def select_bucket(tokens: int, buckets: tuple[int, ...]) -> int:
    """The smallest bucket that holds ``tokens``."""
    if tokens < 1:
        raise ValueError(f"select_bucket needs at least one token, got {tokens}")
    for b in buckets:
        if tokens <= b:
            return b
    raise ValueError(f"no graph bucket holds {tokens} tokens (the largest is {buckets[-1]})")


__all__ = ["KVCache", "get_num_pages", "get_last_page_len", "static_block_table", "graph_buckets",
           "select_bucket", "DRAFT_MODE", "VERIFY_MODE"]
