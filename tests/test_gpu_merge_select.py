"""Split-KV merge and page selection on the GPU."""

from pathlib import Path

import numpy as np
import pytest
import torch

from aspire_amd import _lib
from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper
from aspire_amd.backends.page_selector import KeyMeanPageSelector, PageSelector, PageSelectorFirstLastAvg
from aspire_amd.workloads import PAGE, build_step
from helpers import assert_topk_sets, say
from oracle.attention import paged_attention
from oracle.merge import merge_states
from oracle.select import FirstLastSelector, topk_pages_per_head

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden" / "select_first_last.npz"


@pytest.mark.parametrize("n", [1, 2, 5])
def test_merge_states_matches_oracle(gpu, n):
    say("merge_states", n)
    g = torch.Generator().manual_seed(n)
    rows = 333
    v = torch.randn(n, rows, 128, generator=g)
    s = torch.randn(n, rows, generator=g) * 4
    if n > 1:
        s[1, :7] = float("-inf")
    ref_o, ref_s = merge_states(v, s)
    vd, sd = v.to(gpu), s.to(gpu)
    o32 = torch.empty(rows, 128, device=gpu)
    o16 = torch.empty(rows, 128, device=gpu, dtype=torch.bfloat16)
    so = torch.empty(rows, device=gpu)
    L = _lib.lib()
    st = _lib.stream_of(vd)
    _lib.check(L.aspire_merge_states(_lib.ptr(vd), _lib.ptr(sd), n, rows, 128, _lib.ptr(o32), 0, _lib.ptr(so), st), "m")
    _lib.check(L.aspire_merge_states(_lib.ptr(vd), _lib.ptr(sd), n, rows, 128, _lib.ptr(o16), 1, None, st), "m")
    torch.cuda.synchronize()
    assert torch.allclose(o32.cpu(), ref_o, atol=1e-5, rtol=1e-5)
    assert torch.allclose(so.cpu(), ref_s, atol=1e-5)
    assert torch.allclose(o16.float().cpu(), ref_o, atol=2e-2)


def _golden_case(z, name, gpu, order):
    g = lambda k: z[f"{name}/{k}"]
    B, H, page, max_seq, kv_stride, subset, L, pct, min_pages = g("params").tolist()
    kw = dict(max_batch_size=int(B), pages_per_slot=int(max_seq) // int(page), subset_cache_size=int(subset), L=int(L),
              n_heads=int(H), page_size=int(page), max_seq_length=int(max_seq), device=gpu, bsz=int(B), dec_len=8,
              head_dim=128, kv_stride=int(kv_stride), draft_percent=None if pct < 0 else float(pct),
              min_draft_pages=int(min_pages))
    sel = PageSelectorFirstLastAvg(**kw, order=order)
    dev = lambda a: torch.from_numpy(a).to(gpu)
    inp = dict(attention_weights_buffer=dev(g("dump")).view(torch.float16), lse_buffer=dev(g("lse")),
               num_pages=dev(g("num_pages")), block_table=dev(g("block_table")), qo_indptr=dev(g("qo_indptr")))
    return sel, inp, g


@pytest.mark.parametrize("name", ["small_fixed", "percent", "ties_inf"])
def test_first_last_selector_against_reference_golden(gpu, name):
    say("selector golden", name)
    z = np.load(GOLDEN)
    sel, inp, g = _golden_case(z, name, gpu, "physical")
    selected, valid = sel.select(**inp)
    torch.cuda.synchronize()
    assert np.array_equal(valid.cpu().numpy(), g("valid"))
    ref_scores = g("scores")
    npg = g("num_pages")
    table = g("block_table")
    got_scores = sel._scores.cpu().numpy()
    for b in range(len(npg)):
        n = int(npg[b])
        a, r = got_scores[b, :n], ref_scores[b, :n]
        fin = np.isfinite(r)
        assert np.array_equal(np.isfinite(a), fin)
        assert np.allclose(a[fin], r[fin], rtol=1e-5, atol=1e-6)
        # sets: exact wherever the gap exceeds 1e-3 (forced last-L pages are +inf)
        eff = r.astype(np.float64).copy()
        eff[max(n - int(sel.L), 0) : n] = np.inf
        k = int(g("valid")[b])
        inv = {int(p): j for j, p in enumerate(table[b])}
        got_logical = [inv[int(p)] for p in selected[b, :k].cpu().numpy()]
        assert_topk_sets(got_logical, eff, k)
        row = selected[b].cpu().numpy()
        assert np.all(np.diff(row[:k]) > 0) and not row[k:].any()
        if name != "ties_inf":
            assert np.array_equal(row, g("selected")[b])


@pytest.mark.parametrize("case", ["odd_stride", "misaligned", "odd_length", "page8"])
def test_first_last_generic_scores_kernel(gpu, case):
    """The (R) selector's scores kernel for dumps the 16-byte vector kernel cannot read: a row
    stride that is not a multiple of 8 entries, a dump view 2 bytes past a 16-byte boundary, a
    max_seq_length that is not a multiple of 8, and 8-token pages. Scores equal the reference
    chain (page_selector.py:132-138,163-181) as the oracle restates it; sets are exact wherever
    the score gap exceeds 1e-3. Entries past a row's length are -inf, and some are NaN."""
    say("selector generic scores", case)
    B, H = 3, 8
    page = 8 if case == "page8" else 16
    max_seq = 1004 if case == "odd_length" else 1024
    kv_stride = {"odd_stride": 1028, "odd_length": 1004}.get(case, 1024)
    pages = (max_seq + page - 1) // page
    gen = torch.Generator().manual_seed(12)
    kv_len = [max_seq, 613, 37]
    dump = (torch.randn(B, H, 2, kv_stride, generator=gen) * 6).to(torch.float16)
    for b, n in enumerate(kv_len):
        dump[b, :, :, n:] = float("-inf")
    dump[0, 3, 1, ::41] = float("nan")
    dump[1, :, 0, 200] = float("nan")  # every head NaN for one token
    # per-page key bias so page scores separate
    bias = (torch.randn(B, 1, 1, pages, generator=gen) * 3).repeat_interleave(page, dim=3)[..., :kv_stride]
    dump = (dump.float() + torch.nn.functional.pad(bias, (0, kv_stride - bias.shape[-1]))).to(torch.float16)
    qo = torch.tensor([0, 1, 5, 7], dtype=torch.int32)
    lse = torch.randn(7, H, generator=gen) + 9
    npg = torch.tensor([(n + page - 1) // page for n in kv_len], dtype=torch.int32)
    table = torch.stack([torch.randperm(pages, generator=gen) + b * pages for b in range(B)]).to(torch.int32)
    subset, L = 24, 3
    kw = dict(pages_per_slot=pages, subset_cache_size=subset, L=L, n_heads=H, page_size=page, max_seq_length=max_seq,
              bsz=B, head_dim=128, kv_stride=kv_stride, min_draft_pages=subset)
    flat = dump.reshape(-1)
    if case == "misaligned":
        holder = torch.zeros(flat.numel() + 8, dtype=torch.float16, device=gpu)
        dump_dev = holder[1 : 1 + flat.numel()]
        dump_dev.copy_(flat.to(gpu))
        assert dump_dev.data_ptr() % 16 == 2
    else:
        dump_dev = flat.to(gpu)
    sel = PageSelectorFirstLastAvg(max_batch_size=B, device=gpu, dec_len=8, order="logical", **kw)
    selected, valid = sel.select(dump_dev, lse.to(gpu), npg.to(gpu), table.to(gpu), qo.to(gpu))
    torch.cuda.synchronize()
    ref = FirstLastSelector(**kw)
    ref_scores = ref.page_scores(flat, lse, qo)
    eff = ref.effective_scores(ref_scores, npg)
    got_scores = sel._scores[:B].cpu()
    for b in range(B):
        n = int(npg[b])
        a, r = got_scores[b, :n].numpy(), ref_scores[b, :n].numpy()
        assert np.allclose(a, r, rtol=1e-5, atol=1e-6), (b, np.abs(a - r).max())
        k = int(valid[b])
        assert k == min(n, subset)
        inv = {int(p): j for j, p in enumerate(table[b].numpy())}
        logical = [inv[int(p)] for p in selected[b, :k].cpu().numpy()]
        assert logical == sorted(logical)
        assert_topk_sets(logical, eff[b, :n].double().numpy(), k)


@pytest.mark.parametrize("name", ["small_fixed", "percent", "ties_inf"])
def test_compact_first_last_against_reference_golden(gpu, name):
    """select_from_compact_first_last (page_selector.py:183-184): the dump as a [B, H, 2, seq_len]
    view and the first / last query rows' LSEs given per row select exactly what select() does
    through the token indptr, and match the reference-recorded selections."""
    say("compact selector golden", name)
    z = np.load(GOLDEN)
    sel, inp, g = _golden_case(z, name, gpu, "physical")
    B, H, page, max_seq, kv_stride = (int(x) for x in g("params")[:5])
    qo = g("qo_indptr").astype(np.int64)
    lse = inp["lse_buffer"]
    top = lse.shape[0] - 1
    first = lse[torch.from_numpy(np.clip(qo[:B], 0, top)).to(gpu)]
    last = lse[torch.from_numpy(np.clip(qo[1 : B + 1] - 1, 0, top)).to(gpu)]
    logits = inp["attention_weights_buffer"][: B * H * 2 * kv_stride].view(B, H, 2, kv_stride)[..., :max_seq]
    got, got_valid = (t.clone() for t in sel.select_from_compact_first_last(
        logits, first, last, inp["num_pages"], inp["block_table"]))
    want, want_valid = sel.select(**inp)
    torch.cuda.synchronize()
    assert torch.equal(got, want) and torch.equal(got_valid, want_valid)
    assert np.array_equal(got_valid.cpu().numpy(), g("valid"))
    if name != "ties_inf":
        assert np.array_equal(got.cpu().numpy(), g("selected"))


def test_compact_first_last_layers(gpu):
    """select_layers_from_compact_first_last (page_selector.py:186-204): three layers' dumps in one
    call equal three single-layer calls, and each layer's sets match the oracle wherever the score
    gap exceeds 1e-3; the counts are the first layer's (every layer has the same pages)."""
    say("compact selector, layers")
    n_layers, B, H, page, max_seq = 3, 4, 8, 16, 1024
    kv_stride = 1040
    gen = torch.Generator().manual_seed(17)
    logits = (torch.randn(n_layers, B, H, 2, kv_stride, generator=gen) * 5).to(torch.float16)
    npg = torch.tensor([64, 40, 3, 17], dtype=torch.int32)
    for b, n in enumerate(npg.tolist()):
        logits[:, b, :, :, n * page :] = float("-inf")
    first = torch.randn(n_layers, B, H, generator=gen) + 8
    last = torch.randn(n_layers, B, H, generator=gen) + 8
    table = torch.stack([torch.randperm(64, generator=gen) + 64 * b for b in range(B)]).to(torch.int32)
    kw = dict(max_batch_size=n_layers * B, pages_per_slot=64, subset_cache_size=12, L=2, n_heads=H, page_size=page,
              max_seq_length=max_seq, device=gpu, bsz=B, dec_len=4, kv_stride=kv_stride)
    sel = PageSelectorFirstLastAvg(**kw)
    d = lambda t: t.to(gpu)
    got, valid = (t.clone() for t in sel.select_layers_from_compact_first_last(d(logits), d(first), d(last), d(npg),
                                                                                 d(table)))
    assert got.shape == (n_layers, B, 12) and valid.shape == (B,)
    ref = FirstLastSelector(pages_per_slot=64, subset_cache_size=12, L=2, n_heads=H, page_size=page,
                            max_seq_length=max_seq, bsz=B, kv_stride=kv_stride)
    for layer in range(n_layers):
        one, one_valid = sel.select_from_compact_first_last(d(logits[layer, ..., :max_seq]), d(first[layer]),
                                                            d(last[layer]), d(npg), d(table))
        torch.cuda.synchronize()
        assert torch.equal(got[layer], one) and torch.equal(valid, one_valid), layer
        # the oracle's select() through a token indptr whose first / last rows carry these LSEs
        lse = torch.stack([first[layer], last[layer]], dim=1).reshape(2 * B, H)
        qo = torch.arange(0, 2 * B + 1, 2, dtype=torch.int32)
        scores = ref.page_scores(logits[layer].reshape(-1), lse, qo)
        eff = ref.effective_scores(scores, npg)
        for b in range(B):
            n, k = int(npg[b]), int(valid[b])
            assert k == min(n, 12)
            inv = {int(x): j for j, x in enumerate(table[b].tolist())}
            assert_topk_sets([inv[int(x)] for x in got[layer, b, :k].cpu().tolist()], eff[b, :n].double().numpy(), k)


def test_selector_logical_order_and_subset(gpu):
    z = np.load(GOLDEN)
    sel, inp, g = _golden_case(z, "small_fixed", gpu, "logical")
    selected, valid = sel.select(**inp)
    table = g("block_table")
    for b in range(4):
        k = int(valid[b])
        inv = {int(p): j for j, p in enumerate(table[b])}
        logical = [inv[int(p)] for p in selected[b, :k].cpu().numpy()]
        assert logical == sorted(logical)
    full = selected.clone()
    valid = valid.clone()  # the selector returns views of its preallocated buffers (as the reference does)
    sub, sub_valid = sel.select_subset(torch.tensor([2, 0], device=gpu), **inp)
    torch.cuda.synchronize()
    assert torch.equal(sub[0], full[2]) and torch.equal(sub[1], full[0])
    assert sub_valid.tolist() == [int(valid[2]), int(valid[0])]


def test_last_token_selector_matches_torch_chain(gpu):
    say("last-token selector")
    B, H, page, max_seq = 3, 8, 16, 1024
    gen = torch.Generator().manual_seed(4)
    dump = (torch.randn(B, H, max_seq, generator=gen) * 5).to(torch.float16)
    dump[1, :, 600:] = float("-inf")
    lse = torch.randn(6, H, generator=gen) + 7
    npg = torch.tensor([64, 38, 5], dtype=torch.int32)
    table = torch.arange(B * 64, dtype=torch.int32).view(B, 64)
    qo = torch.tensor([0, 2, 3, 6, 6], dtype=torch.int32)
    sel = PageSelector(B, 64, 10, 2, H, page, max_seq, gpu, B, 4, min_draft_pages=10)
    selected, valid = sel.select(dump.view(-1).to(gpu), lse.to(gpu), npg.to(gpu), table.to(gpu), qo.to(gpu))
    torch.cuda.synchronize()
    # the reference's last-token chain (page_selector.py:110-130), restated with torch on the CPU
    last = (qo[1 : B + 1].long() - 1).clamp(min=0)
    norm = dump.float() * 0 + (dump * sel._sm_scale_log2e).float() - lse[last][:, :, None]
    norm.nan_to_num_(nan=float("-inf"))
    tok = torch.exp2(norm.amax(dim=1))
    scores = tok.view(B, 64, 16).sum(-1) - torch.arange(64, dtype=torch.float32) * 1e-7
    for b in range(B):
        n = int(npg[b])
        eff = scores[b, :n].double().numpy().copy()
        eff[max(n - 2, 0) :] = np.inf
        k = min(n, 10)
        assert int(valid[b]) == k
        assert_topk_sets((selected[b, :k].cpu().numpy() - b * 64).tolist(), eff, k)


def test_keymean_selector_config2_shape(gpu):
    say("key-mean selector")
    step = build_step(hq=32, hkv=8, ctx_len=[8192, 9000, 12000, 8200], q_len=[1] * 4, is_draft=[0] * 4,
                      draft_budget=0, seed=21, device=gpu)
    w = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD")
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 32, 8, 128, PAGE, causal=True)
    max_pages = int(step.block_table.shape[1])
    ks = KeyMeanPageSelector(4, 8, max_pages, k=128, L=0, device=gpu)
    ks.page_scores.fill_(float("nan"))
    w.run(step.q, step.cache, page_scores=ks.page_scores)
    npg = torch.from_numpy((step.ctx_len + 15) // 16).to(torch.int32).to(gpu)
    selected, counts = ks.select(npg, step.block_table)
    torch.cuda.synchronize()
    ref_scores = torch.full((4 * 8, max_pages), float("nan"))
    paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host, step.kv_indices.cpu(),
                    step.kv_len_host, num_kv_heads=8, page_scores=ref_scores)
    table = step.block_table.cpu().numpy()
    for b in range(4):
        n = int(npg[b])
        inv = {int(p): j for j, p in enumerate(table[b, :n])}
        for g in range(8):
            k = int(counts[b, g])
            assert k == min(128, n)
            logical = [inv[int(p)] for p in selected[b, g, :k].cpu().numpy()]
            assert logical == sorted(logical)
            assert_topk_sets(logical, ref_scores[b * 8 + g, :n].double().numpy(), k)


def _topk_expected(scores, n, L, kk, table_row, order):
    """Top-kk of one segment: +inf for the last L pages, ties by lowest index, ascending logical."""
    sc = scores[:n].astype(np.float32).copy()
    if L > 0:
        sc[max(n - L, 0):] = np.inf
    u = sc.view(np.uint32).astype(np.int64)
    key = np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)
    pick = np.sort(np.argsort(-key, kind="stable")[:kk])
    phys = table_row[pick]
    return np.sort(phys) if order == 0 else phys


@pytest.mark.parametrize("order", [0, 1])
@pytest.mark.parametrize("stride", [12288, 2048, 700])
def test_topk_kernel_exact_with_ties_and_wide_rows(gpu, order, stride):
    """Keys in LDS (stride > 2048) and in registers (stride <= 2048); counts above the stride are clamped."""
    say("topk exact", order, stride)
    rng = np.random.default_rng(11 + order)
    segs = 8
    npg = np.array([12288, 5000, 300, 64, 1, 0, 2049, 230], dtype=np.int32)
    # coarse values -> many exact ties; a few +-inf
    scores = (rng.integers(-40, 40, size=(segs, stride)) * 0.25).astype(np.float32)
    scores[1, ::97] = np.inf
    scores[2, :50] = -np.inf
    table = np.stack([rng.permutation(stride).astype(np.int32) for _ in range(segs)])
    L, subset, width = 3, 1500, 1800
    sel = torch.full((segs, width), -1, dtype=torch.int32, device=gpu)
    valid = torch.zeros(segs, dtype=torch.int32, device=gpu)
    sd, nd, td = (torch.from_numpy(a).to(gpu) for a in (scores, npg, table))
    _lib.check(_lib.lib().aspire_select_topk(_lib.ptr(sd), stride, _lib.ptr(nd), None, segs, 1, L, 0, subset, 0, 0.0,
                                             _lib.ptr(td), stride, order, _lib.ptr(sel), width, width,
                                             _lib.ptr(valid), _lib.stream_of(sd)), "topk")
    torch.cuda.synchronize()
    got, got_valid = sel.cpu().numpy(), valid.cpu().numpy()
    for s in range(segs):
        n = min(int(npg[s]), stride)
        k = min(n, subset)
        assert got_valid[s] == k
        exp = _topk_expected(scores[s], n, L, k, table[s], order)
        assert np.array_equal(got[s, :k], exp), s
        assert not got[s, k:].any()


@pytest.mark.parametrize("order", [0, 1])
def test_topk_kernel_radix_digits(gpu, order):
    """Key sets that walk every digit of the radix select (rows of up to 2,048 pages): keys
    that differ only in their low 10 bits, ties straddling the k-th key in each digit, an
    all-equal row, signed zeros, negative-only rows, the forced last pages, and budgets of
    0, 1, n - 1 and n."""
    say("topk radix digits", order)
    rng = np.random.default_rng(23 + order)
    stride = 2048
    base = np.float32(1.0)
    ulps = (base.view(np.uint32) + np.arange(stride, dtype=np.uint32)).view(np.float32)
    rows = [
        rng.permutation(ulps),                                       # keys differ in bits 0..10 only
        np.repeat(rng.permutation(ulps[:64]), 32),                   # 32-fold ties, low bits
        np.full(stride, 3.5, dtype=np.float32),                      # one value
        rng.choice(np.array([0.0, -0.0, 1e-30, -1e-30], dtype=np.float32), stride),
        -np.abs(rng.standard_normal(stride)).astype(np.float32),     # negative only
        (rng.integers(0, 3, stride) * np.float32(2.0) ** 20).astype(np.float32),  # ties in the top digit
        rng.standard_normal(stride).astype(np.float32),
        (ulps * np.where(rng.random(stride) < 0.5, 1, 1024)).astype(np.float32),  # two clusters
    ]
    scores = np.stack(rows).astype(np.float32)
    segs = scores.shape[0]
    table = np.stack([rng.permutation(stride).astype(np.int32) for _ in range(segs)])
    sd, td = (torch.from_numpy(a).to(gpu) for a in (scores, table))
    for npg_list, L, subset in (([2048, 2048, 2048, 2048, 2048, 2048, 2048, 2048], 0, 128),
                                ([2048, 1700, 513, 2000, 1999, 2048, 1024, 777], 5, 700),
                                ([2048, 2, 1, 2048, 3, 129, 2048, 64], 0, 2047),
                                ([128, 2048, 16, 1000, 2048, 2048, 1, 100], 2, 1)):
        npg = np.array(npg_list, dtype=np.int32)
        width = subset
        sel = torch.full((segs, width), -1, dtype=torch.int32, device=gpu)
        valid = torch.zeros(segs, dtype=torch.int32, device=gpu)
        nd = torch.from_numpy(npg).to(gpu)
        _lib.check(_lib.lib().aspire_select_topk(_lib.ptr(sd), stride, _lib.ptr(nd), None, segs, 1, L, 0, subset, 0,
                                                 0.0, _lib.ptr(td), stride, order, _lib.ptr(sel), width, width,
                                                 _lib.ptr(valid), _lib.stream_of(sd)), "topk")
        torch.cuda.synchronize()
        got, got_valid = sel.cpu().numpy(), valid.cpu().numpy()
        for s in range(segs):
            n = int(npg[s])
            k = min(n, subset)
            assert got_valid[s] == k
            exp = _topk_expected(scores[s], n, L, k, table[s], order)
            assert np.array_equal(got[s, :k], exp), (npg_list, s)
            assert not got[s, k:].any()


def test_topk_kernel_width_clamp_and_percent_count(gpu):
    rng = np.random.default_rng(5)
    segs, stride = 4, 4096
    npg = np.array([4096, 1000, 17, 3], dtype=np.int32)
    scores = rng.standard_normal((segs, stride)).astype(np.float32)
    table = np.tile(np.arange(stride, dtype=np.int32), (segs, 1))
    width, pct, lo, hi = 64, 7.0, 20, 400
    sel = torch.full((segs, width), -1, dtype=torch.int32, device=gpu)
    valid = torch.zeros(segs, dtype=torch.int32, device=gpu)
    sd, nd, td = (torch.from_numpy(a).to(gpu) for a in (scores, npg, table))
    _lib.check(_lib.lib().aspire_select_topk(_lib.ptr(sd), stride, _lib.ptr(nd), None, segs, 1, 0, 2, hi, lo, pct,
                                             _lib.ptr(td), stride, 0, _lib.ptr(sel), width, width,
                                             _lib.ptr(valid), _lib.stream_of(sd)), "topk")
    torch.cuda.synchronize()
    for s in range(segs):
        n = int(npg[s])
        k = min(max(int(np.ceil(np.float32(n) * np.float32(pct) / np.float32(100.0))), min(n, lo)), min(n, hi))
        assert int(valid[s]) == k
        kk = min(k, width)
        assert np.array_equal(sel[s, :kk].cpu().numpy(), _topk_expected(scores[s], n, 0, kk, table[s], 0))


def test_selectors_graph_replays_match_eager(gpu):
    """Both selectors captured in a HIP graph (as the reference replays them): every replay equals eager."""
    say("selector graph replays")
    z = np.load(GOLDEN)
    sel, inp, g = _golden_case(z, "percent", gpu, "physical")
    eager_sel, eager_valid = (t.clone() for t in sel.select(**inp))
    step = build_step(hq=32, hkv=8, ctx_len=[3000, 4096, 700], q_len=[1] * 3, is_draft=[0] * 3,
                      draft_budget=0, seed=3, device=gpu)
    npg = torch.from_numpy((step.ctx_len + 15) // 16).to(torch.int32).to(gpu)
    ks = KeyMeanPageSelector(3, 8, int(step.block_table.shape[1]), k=64, L=2, device=gpu)
    ks.page_scores.copy_(torch.randn(ks.page_scores.shape, generator=torch.Generator(device=gpu).manual_seed(1),
                                     device=gpu))
    k_sel, k_cnt = (t.clone() for t in ks.select(npg, step.block_table))
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sel.select(**inp)
        ks.select(npg, step.block_table)
    for rep in range(3):
        sel._selected_buf.fill_(-7)
        ks.selected.fill_(-7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got_sel, got_valid = sel._selected_buf[: eager_sel.shape[0], : eager_sel.shape[1]], sel._valid_counts_buf
        assert torch.equal(got_sel, eager_sel), rep
        assert torch.equal(got_valid[: eager_valid.numel()], eager_valid), rep
        assert torch.equal(ks.selected[:3], k_sel) and torch.equal(ks.counts[:3], k_cnt), rep
