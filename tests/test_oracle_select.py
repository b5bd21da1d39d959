"""The CPU selector oracle against the reference's own outputs and special cases."""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.select import FirstLastSelector, topk_pages_per_head

GOLDEN = Path(__file__).resolve().parent / "golden" / "select_first_last.npz"


def _load_case(z, name):
    g = lambda k: z[f"{name}/{k}"]
    B, H, page, max_seq, kv_stride, subset, L, pct, min_pages = g("params").tolist()
    sel = FirstLastSelector(
        pages_per_slot=int(max_seq) // int(page), subset_cache_size=int(subset), L=int(L), n_heads=int(H),
        page_size=int(page), max_seq_length=int(max_seq), bsz=int(B), head_dim=128, kv_stride=int(kv_stride),
        draft_percent=None if pct < 0 else float(pct), min_draft_pages=int(min_pages),
    )
    inputs = dict(
        dump_flat=torch.from_numpy(g("dump")).view(torch.float16),
        lse_buffer=torch.from_numpy(g("lse")),
        num_pages=torch.from_numpy(g("num_pages")),
        block_table=torch.from_numpy(g("block_table")),
        qo_indptr=torch.from_numpy(g("qo_indptr")),
    )
    return sel, inputs, g


@pytest.mark.parametrize("name", ["small_fixed", "percent", "ties_inf"])
def test_first_last_selector_matches_reference_golden(name):
    z = np.load(GOLDEN)
    sel, inp, g = _load_case(z, name)
    scores = sel.page_scores(inp["dump_flat"], inp["lse_buffer"], inp["qo_indptr"])
    # Same torch ops on the same CPU: the page scores are bit-identical.
    assert torch.equal(scores, torch.from_numpy(g("scores")))
    selected, valid = sel.finalize(scores, inp["num_pages"], inp["block_table"], order="physical")
    assert torch.equal(valid, torch.from_numpy(g("valid")))
    assert torch.equal(selected, torch.from_numpy(g("selected")))


def test_logical_order_equals_physical_for_increasing_table():
    z = np.load(GOLDEN)
    sel, inp, g = _load_case(z, "percent")  # arange table
    a, va = sel.select(**inp, order="physical")
    b, vb = sel.select(**inp, order="logical")
    assert torch.equal(a, b) and torch.equal(va, vb)


def test_one_hot_dump_selects_the_hot_page():
    # Every logit -inf except one token in page 5 of row 0 (both slots): the
    # hot page must be selected alongside the forced last L pages.
    B, H, page, max_seq = 1, 4, 16, 256
    sel = FirstLastSelector(pages_per_slot=16, subset_cache_size=3, L=2, n_heads=H, page_size=page,
                            max_seq_length=max_seq, bsz=B, min_draft_pages=3)
    dump = torch.full((B, H, 2, max_seq), float("-inf"), dtype=torch.float16)
    dump[0, 1, :, 5 * 16 + 7] = 10.0
    lse = torch.zeros(2, H)
    qo = torch.tensor([0, 2, 2], dtype=torch.int32)
    sel_pages, valid = sel.select(dump.view(-1), lse, torch.tensor([16], dtype=torch.int32),
                                  torch.arange(16, dtype=torch.int32).view(1, 16), qo)
    assert valid.tolist() == [3]
    assert sel_pages[0].tolist() == [5, 14, 15]


def test_all_pages_when_budget_exceeds_pages():
    sel = FirstLastSelector(pages_per_slot=8, subset_cache_size=8, L=2, n_heads=2, page_size=16,
                            max_seq_length=128, bsz=1, min_draft_pages=8)
    dump = torch.randn(1, 2, 2, 128).to(torch.float16)
    table = torch.tensor([[7, 3, 5, 1, 0, 2, 6, 4]], dtype=torch.int32)
    s, v = sel.select(dump.view(-1), torch.zeros(1, 2), torch.tensor([5], dtype=torch.int32), table,
                      torch.tensor([0, 1, 1], dtype=torch.int32))
    assert v.tolist() == [5]
    assert s[0, :5].tolist() == sorted([7, 3, 5, 1, 0]) and s[0, 5:].tolist() == [0, 0, 0]


def test_valid_counts_percent_rule():
    sel = FirstLastSelector(pages_per_slot=2048, subset_cache_size=144, L=8, n_heads=2, page_size=16,
                            max_seq_length=32768, bsz=1, draft_percent=7.0, min_draft_pages=32)
    npg = torch.tensor([0, 5, 32, 100, 457, 2048], dtype=torch.int32)
    want = [min(max(math.ceil(n * 0.07), min(n, 32)), min(n, 144)) for n in npg.tolist()]
    assert sel.compute_valid_counts(npg).tolist() == want


def test_keymean_topk_brute_force():
    g = torch.Generator().manual_seed(3)
    scores = torch.randn(6, 40, generator=g)
    npg = torch.tensor([40, 39, 5, 0, 17, 33])
    idx, cnt = topk_pages_per_head(scores, npg, k=8, L=1)
    for s in range(6):
        n = int(npg[s])
        expect = set()
        if n:
            expect.add(n - 1)
            rest = sorted(range(n - 1), key=lambda j: -float(scores[s, j]))
            expect.update(rest[: min(8, n) - 1])
        assert cnt[s] == min(8, n)
        assert idx[s, : cnt[s]].tolist() == sorted(expect)
