"""The decode-step oracle: row operations by closed forms, the composed step by invariants
that a wrong list, length or index would break."""

import math

import numpy as np
import torch

from aspire_amd.decode_step import DecodeWeights, ModelShape
from aspire_amd.workloads import random_block_table
from oracle.decode import add_rms_norm, argmax_rows, decode_step, silu_mul


def test_add_rms_norm_closed_forms():
    w = (torch.rand(256) + 0.5).to(torch.bfloat16)
    x = torch.full((2, 256), 1.5, dtype=torch.bfloat16)
    d = torch.full((2, 256), 0.5, dtype=torch.bfloat16)
    x2, out = add_rms_norm(x, w, 1e-6, d)
    assert torch.equal(x2, torch.full((2, 256), 2.0, dtype=torch.bfloat16))   # 1.5 + 0.5 exactly
    assert torch.equal(out, w.expand(2, 256))                                   # constant row -> the weight
    # a row (a, -a, a, -a ...) has mean square a^2: every entry becomes +-1 times the weight
    x = torch.tensor([3.0, -3.0] * 128, dtype=torch.bfloat16).view(1, 256)
    _, out = add_rms_norm(x, w, 0.0)
    assert torch.equal(out[0], (w.float() * torch.tensor([1.0, -1.0] * 128)).to(torch.bfloat16))


def test_silu_mul_against_fp64():
    g = torch.linspace(-12, 12, 512).to(torch.bfloat16)
    u = torch.linspace(3, -2, 512).to(torch.bfloat16)
    out = silu_mul(torch.cat([g, u]).view(1, 1024))[0].double()
    gd, ud = g.double(), u.double()
    silu = gd / (1 + torch.exp(-gd))
    exact = silu.to(torch.bfloat16).double() * ud
    # one bf16 rounding of the product: within half an ulp (2^-8 relative)
    assert torch.all((out - exact).abs() <= exact.abs() * 2.0 ** -8 + 1e-30)
    assert out[torch.argmin(gd.abs())].abs() <= 0.03     # silu(~0) = ~0
    big = gd > 10
    assert torch.allclose(out[big], (gd[big] * ud[big]).to(torch.bfloat16).double(), rtol=1e-2)


def test_argmax_first_index_of_ties():
    x = torch.zeros(2, 10, dtype=torch.bfloat16)
    x[0, 3] = x[0, 7] = 5.0
    x[1, :] = float("-inf")
    x[1, 9] = -1.0
    assert argmax_rows(x).tolist() == [3, 9]


SHAPE = ModelShape(n_layer=3, dim=256, n_head=4, n_local_heads=2, head_dim=128, intermediate_size=512,
                   vocab_size=64, rope_base=1e6)


def _setup(seed=0):
    w = DecodeWeights(SHAPE, "cpu", seed=seed)
    ctx = np.array([70, 130, 33])
    ql = np.array([1, 4, 1])
    dr = np.array([True, False, True])
    n_pages = (ctx + 15) // 16
    table, pool = random_block_table(n_pages, seed=seed, pool_pages=int(n_pages.sum()) + 5)
    g = torch.Generator().manual_seed(seed)
    caches = torch.randn(SHAPE.n_layer, pool, 2, 16, 2, 128, generator=g).to(torch.bfloat16)
    tokens = torch.randint(0, SHAPE.vocab_size, (int(ql.sum()),), generator=g)
    return w, ctx, ql, dr, n_pages, table, caches, tokens


def _full_selection(n_pages, table, budget):
    B, H = len(n_pages), SHAPE.n_local_heads
    sel = np.zeros((B, H, budget), dtype=np.int64)
    cnt = np.zeros((B, H), dtype=np.int64)
    for b in range(B):
        c = min(budget, int(n_pages[b]))
        sel[b, :, :c] = table[b, n_pages[b] - c : n_pages[b]]
        cnt[b] = c
    return sel, cnt


def test_step_with_every_page_selected_ignores_the_refresh_layer():
    """A budget covering every page makes each draft segment its full row list, so the
    logits cannot depend on which layer refreshes (a wrong per-head length, list or
    selection rule would make them differ)."""
    w, ctx, ql, dr, n_pages, table, caches, tokens = _setup()
    budget = int(n_pages.max())
    sel, cnt = _full_selection(n_pages, table, budget)
    kw = dict(budget=budget, recent_pages=1, selected=sel, counts=cnt)
    a = decode_step(w, caches.clone(), SHAPE, ctx, ql, dr, table, tokens, refresh_layer=0, **kw)
    b = decode_step(w, caches.clone(), SHAPE, ctx, ql, dr, table, tokens, refresh_layer=2, **kw)
    assert torch.equal(a["logits"], b["logits"])
    for bb in np.flatnonzero(dr):
        assert a["selected_counts"][bb].tolist() == [n_pages[bb]] * 2


def test_step_is_invariant_under_a_pool_permutation():
    """Relabelling the physical pages (table and caches together) changes nothing."""
    w, ctx, ql, dr, n_pages, table, caches, tokens = _setup(1)
    budget = 3
    sel, cnt = _full_selection(n_pages, table, budget)
    kw = dict(budget=budget, recent_pages=1, refresh_layer=1)
    a = decode_step(w, caches.clone(), SHAPE, ctx, ql, dr, table, tokens, selected=sel, counts=cnt, **kw)
    perm = np.random.default_rng(5).permutation(caches.shape[1])
    inv = np.argsort(perm)                      # new page id of old page p is inv[p]
    caches2 = caches[:, torch.from_numpy(perm)].clone()
    table2 = inv[table]
    sel2 = np.where(np.arange(budget)[None, None, :] < cnt[..., None], inv[sel], 0)
    b = decode_step(w, caches2, SHAPE, ctx, ql, dr, table2, tokens, selected=sel2, counts=cnt, **kw)
    assert torch.equal(a["logits"], b["logits"])
    assert np.array_equal(a["selected_logical"], b["selected_logical"])
    assert not math.isnan(float(a["logits"].float().abs().max()))
