"""Layout owners (cache views, page math, block table, graph buckets) against worked values."""

import pytest
import torch

from aspire_amd.attention.layout import (DRAFT_MODE, VERIFY_MODE, KVCache, get_last_page_len, get_num_pages,
                                         graph_buckets, select_bucket, static_block_table)


def test_page_math_documented_examples():
    # mixed_runner.py:98-120 docstring: page 128 -> seq 1 -> 1, 128 -> 128, 129 -> 1; empty -> 0
    lens = torch.tensor([1, 128, 129, 0, 256], dtype=torch.int32)
    assert get_last_page_len(lens, 128).tolist() == [1, 128, 1, 0, 128]
    assert get_num_pages(lens, 128).tolist() == [1, 1, 2, 0, 2]


def test_unified_cache_views_share_storage():
    c = KVCache(6, 16, 8, 128, spec=True, draft_max_num_pages=3)
    assert c.unified_cache.shape == (9, 2, 16, 8, 128) and c.kv_cache.shape[0] == 6 and c.draft_cache.shape[0] == 3
    c.draft_cache[0, 1, 5, 2, 7] = 3.0  # V of draft page 0 is unified page 6
    assert c.unified_cache[6, 1, 5, 2, 7].item() == 3.0
    assert c.kv_cache.data_ptr() == c.unified_cache.data_ptr()
    plain = KVCache(4, 16, 8, 128)
    assert plain.unified_cache is plain.kv_cache and plain.kv_cache.shape == (4, 2, 16, 8, 128)


def test_static_block_table():
    t, per, total = static_block_table(3, 100, 16)  # 100 tokens -> 6 whole pages, plus one per request
    assert (per, total) == (7, 21) and t.shape == (3, 7)
    assert t[2].tolist() == list(range(14, 21))
    t, per, total = static_block_table(2, 64, 16)
    assert (per, total) == (4, 8)


def test_graph_buckets():
    assert graph_buckets(1) == (1,)
    assert graph_buckets(20) == (1, 2, 4, 8, 16, 20)
    assert graph_buckets(24) == (1, 2, 4, 8, 16, 24)
    b = graph_buckets(80)
    assert select_bucket(3, b) == 4 and select_bucket(9, b) == 16 and select_bucket(80, b) == 80
    with pytest.raises(ValueError):
        select_bucket(81, b)
    with pytest.raises(ValueError):
        graph_buckets(0)
    assert (DRAFT_MODE, VERIFY_MODE) == (0, 1)
