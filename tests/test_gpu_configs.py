"""BASELINE configs 2 and 4 at their real workloads, the (R) selector at refresh-layer scale,
and masking of stale cache slots past each row's length, on the GPU against the CPU oracle.

Config 2 (workloads.config2): the B=64 refresh layer, contexts
U[8192, 32768], full attention for 64 single-query rows with the per-KV-head key-mean page
scores, top-128 pages per (row, kv head). Config 4 (workloads.config4, configs[4]): batch 16
over 64k-128k contexts at every draft fraction the config sweeps. Sampled rows are checked
against the oracle after their pages are gathered on the device; properties that need no
oracle (finite output, the exact top-k of the GPU's own scores) are checked on every row.
"""

import numpy as np
import pytest
import torch

from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper, build_holistic_dump_jit_args
from aspire_amd.backends.page_selector import KeyMeanPageSelector, PageSelectorFirstLastAvg
from aspire_amd.workloads import PAGE, build_step, config2, config4
from helpers import assert_topk_sets, attn_close, oracle_row, say
from oracle.attention import DumpSpec, paged_attention
from oracle.select import FirstLastSelector

pytestmark = pytest.mark.gpu


def make_wrapper(gpu, **kw):
    return HolisticAttentionWrapper(torch.empty(1, dtype=torch.uint8, device=gpu), "NHD", **kw)


def plan(w, step, causal=True):
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, step.hq, step.hkv, 128, PAGE,
           causal=causal)


def row_pages(step, b):
    kvp = step.kv_indptr_host.numpy()
    return step.kv_indices[int(kvp[b]) : int(kvp[b + 1])].cpu().numpy()


def row_tokens(step, b):
    qo = step.qo_indptr_host.numpy()
    return range(int(qo[b]), int(qo[b + 1]))


def topk_keys(scores: np.ndarray) -> np.ndarray:
    """Order-preserving integer keys of fp32 scores (the selection kernel's total order)."""
    u = scores.astype(np.float32).view(np.uint32).astype(np.int64)
    return np.where(u & 0x80000000, (~u) & 0xFFFFFFFF, u | 0x80000000)


def exact_topk(scores: np.ndarray, n: int, k: int, L: int) -> np.ndarray:
    """The k best of the first n scores (last L forced in; ties to the lower page), ascending."""
    sc = scores[:n].astype(np.float32).copy()
    if L > 0:
        sc[max(n - L, 0) :] = np.inf
    return np.sort(np.argsort(-topk_keys(sc), kind="stable")[:k])


def test_config2_refresh_layer_real_workload(gpu):
    say("config2 real workload: B=64 refresh layer, contexts U[8192, 32768]")
    torch.cuda.empty_cache()
    step = config2(device=gpu)
    B, H, HKV = step.batch, step.hq, step.hkv
    assert B == 64 and H == 32 and HKV == 8
    assert step.ctx_len.min() >= 8192 and step.ctx_len.max() <= 32768
    w = make_wrapper(gpu)
    plan(w, step)
    max_pages = int(step.block_table.shape[1])
    ks = KeyMeanPageSelector(B, HKV, max_pages, k=128, L=0, device=gpu)
    ks.page_scores.fill_(float("nan"))
    out, lse = w.run(step.q, step.cache, return_lse=True, page_scores=ks.page_scores)
    npg_host = (step.ctx_len + PAGE - 1) // PAGE
    npg = torch.from_numpy(npg_host.astype(np.int32)).to(gpu)
    selected, counts = ks.select(npg, step.block_table)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()

    # every (row, kv head): scores written exactly for the row's pages, and the selection is the
    # exact top-128 of the GPU's own scores in ascending logical order
    scores = ks.page_scores.cpu().numpy()
    sel = selected.cpu().numpy()
    cnt = counts.cpu().numpy()
    table = step.block_table.cpu().numpy()
    for b in range(B):
        n = int(npg_host[b])
        for g in range(HKV):
            s = b * HKV + g
            assert np.isfinite(scores[s, :n]).all() and np.isnan(scores[s, n:]).all(), (b, g)
            assert cnt[b, g] == min(128, n)
            want = table[b, exact_topk(scores[s], n, 128, 0)]
            assert np.array_equal(sel[b, g, : cnt[b, g]], want), (b, g)

    # sampled rows against the oracle: output, LSE, page scores, and the selected set under the
    # 1e-3 gap rule on the oracle's scores
    rng = np.random.default_rng(2)
    order = np.argsort(step.ctx_len)
    rows = sorted(set([int(order[0]), int(order[1]), int(order[-1]), int(order[-2])] +
                      rng.choice(B, 4, replace=False).tolist()))
    for b in rows:
        say(f"config2 row {b} ctx {int(step.ctx_len[b])}")
        n = int(npg_host[b])
        ref_scores = torch.full((HKV, n), float("nan"))
        ref_out, ref_lse = oracle_row(step.q, step.cache, row_tokens(step, b), row_pages(step, b),
                                      [int(step.kv_len_host[b])], HKV, page_scores=ref_scores)
        toks = list(row_tokens(step, b))
        attn_close(out[toks], ref_out)
        assert (lse[toks].cpu() - ref_lse).abs().max() < 2e-3
        got = torch.from_numpy(scores[b * HKV : (b + 1) * HKV, :n])
        assert torch.allclose(got, ref_scores, rtol=1e-4, atol=1e-4), b
        inv = {int(p): j for j, p in enumerate(table[b, :n])}
        for g in range(HKV):
            logical = [inv[int(p)] for p in sel[b, g, : cnt[b, g]]]
            assert_topk_sets(logical, ref_scores[g].double().numpy(), int(cnt[b, g]))
    del step, w, ks, out, lse
    torch.cuda.empty_cache()


@pytest.mark.parametrize("frac", [0.0, 0.25, 0.5, 0.75, 1.0])
def test_config4_every_draft_fraction(gpu, frac):
    """Contexts of 64k-128k tokens, verify q_len U{2..9} (all three row-tile classes), 256-page
    drafts: long split-KV chains merged across many pieces, at each swept draft fraction."""
    say(f"config4 draft fraction {frac}")
    torch.cuda.empty_cache()
    step = config4(device=gpu, draft_frac=frac)
    w = make_wrapper(gpu)
    plan(w, step)
    info = w.plan_info
    assert info.num_merge > 0
    rows_per_q = step.q_len * (step.hq // step.hkv)
    for c in range(3):
        present = bool(np.any((rows_per_q > 16 * c) & (rows_per_q <= 16 * (c + 1))))
        assert (info.num_items[c] > 0) == present, (c, list(info.num_items))
    out, lse = w.run(step.q, step.cache, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    drafts = np.flatnonzero(step.is_draft)
    verify = np.flatnonzero(~step.is_draft)
    rows = []
    if drafts.size:
        rows += [int(drafts[0]), int(drafts[-1])]
    if verify.size:
        by_q = verify[np.argsort(step.q_len[verify], kind="stable")]
        rows += [int(by_q[0]), int(by_q[len(by_q) // 2]), int(by_q[-1])]  # smallest, middle, largest q_len
    for b in sorted(set(rows)):
        say(f"config4 f={frac} row {b} q_len {int(step.q_len[b])} ctx {int(step.ctx_len[b])}")
        ref_out, ref_lse = oracle_row(step.q, step.cache, row_tokens(step, b), row_pages(step, b),
                                      [int(step.kv_len_host[b])], step.hkv)
        toks = list(row_tokens(step, b))
        attn_close(out[toks], ref_out)
        assert (lse[toks].cpu() - ref_lse).abs().max() < 2e-3, b
    del step, w, out, lse
    torch.cuda.empty_cache()


def test_first_last_selector_refresh_scale(gpu):
    """The reference (R) selector at refresh-layer scale: 64 rows x 32 heads x 2 slots over a
    32k stride, contexts U[8192, 32768], 7% draft budget with a floor of 32 pages and the last
    8 pages forced, a random-permutation block table, the reference's physical order."""
    say("(R) selector at refresh scale")
    B, H, max_seq = 64, 32, 32768
    rng = np.random.default_rng(17)
    ctx = rng.integers(8192, 32769, size=B)
    npg_host = (ctx + PAGE - 1) // PAGE
    gen = torch.Generator(device=gpu).manual_seed(7)
    dump = (torch.randn(B, H, 2, max_seq, generator=gen, device=gpu) * 6).to(torch.float16)
    pos = torch.arange(max_seq, device=gpu)
    ctx_d = torch.from_numpy(ctx).to(gpu)
    dump.masked_fill_(pos[None, None, None, :] >= ctx_d[:, None, None, None], float("-inf"))
    qlens = rng.integers(1, 10, size=B)
    qo_host = np.concatenate([[0], np.cumsum(qlens)]).astype(np.int32)
    lse = torch.randn(int(qo_host[-1]), H, generator=gen, device=gpu) + 8
    qo = torch.from_numpy(qo_host).to(gpu)
    table = torch.from_numpy(rng.permutation(B * 2048).astype(np.int32).reshape(B, 2048)).to(gpu)
    npg = torch.from_numpy(npg_host.astype(np.int32)).to(gpu)
    kw = dict(pages_per_slot=2048, subset_cache_size=144, L=8, n_heads=H, page_size=PAGE, max_seq_length=max_seq,
              bsz=B, head_dim=128, draft_percent=7.0, min_draft_pages=32)
    sel = PageSelectorFirstLastAvg(max_batch_size=B, device=gpu, dec_len=9, order="physical", **kw)
    selected, valid = sel.select(dump.view(-1), lse, npg, table, qo)
    torch.cuda.synchronize()
    ref = FirstLastSelector(**kw)
    scores = ref.page_scores(dump.view(-1).cpu(), lse.cpu(), torch.from_numpy(qo_host))
    ref_sel, ref_valid = ref.finalize(scores, npg.cpu(), table.cpu(), order="physical")
    eff = ref.effective_scores(scores, npg.cpu())
    assert torch.equal(valid.cpu(), ref_valid)
    got_scores = sel._scores[:B].cpu()
    for b in range(B):
        n = int(npg_host[b])
        assert torch.allclose(got_scores[b, :n], scores[b, :n], rtol=1e-4, atol=1e-6), b
        k = int(valid[b])
        phys = selected[b, :k].cpu().numpy()
        assert np.all(np.diff(phys) > 0), b                     # ascending physical ids
        inv = {int(p): j for j, p in enumerate(table[b, :n].cpu().numpy())}
        assert_topk_sets([inv[int(p)] for p in phys], eff[b, :n].double().numpy(), k)
        assert (selected[b, k:].cpu() == 0).all()
    agree = sum(int(torch.equal(selected[b, : int(valid[b])].cpu(), ref_sel[b, : int(valid[b])]))
                for b in range(B))
    assert agree >= B - 4, f"only {agree} of {B} rows equal the oracle's list exactly"


# ------------------------------------------------------------------ stale slots past kv_len
def _poison_tails(cache: torch.Tensor, step) -> int:
    """Fill every cache slot past each row's length on its current (last) page: K with NaN,
    V with +inf. Returns the number of poisoned pages."""
    table = step.block_table.cpu().numpy()
    n = 0
    for b in range(step.batch):
        ctx = int(step.ctx_len[b])
        last = (ctx - 1) % PAGE + 1
        if last == PAGE:
            continue
        page = int(table[b, (ctx - 1) // PAGE])
        cache[page, 0, last:] = float("nan")
        cache[page, 1, last:] = float("inf")
        n += 1
    return n


TAIL_CASES = [
    # name, hq, hkv, ctx (tails of 1..15 valid keys), q_len, draft
    ("tile1_staged", 32, 8, [1 + 16 * 40, 7 + 16 * 3, 15 + 16 * 100, 2], [1, 4, 2, 1], [1, 0, 0, 0]),
    ("tile2_staged", 32, 8, [1 + 16 * 60, 9 + 16 * 7, 3 + 16 * 200], [5, 8, 6], [0, 0, 0]),
    ("tile3_direct", 32, 8, [1 + 16 * 33, 12 + 16 * 300, 5 + 16 * 2], [9, 12, 10], [0, 0, 0]),
    ("gqa2_mixed", 16, 8, [1 + 16 * 80, 6 + 16 * 20, 13 + 16 * 5], [1, 7, 16], [1, 0, 0]),
    ("hkv2_direct", 8, 2, [1 + 16 * 50, 11 + 16 * 9], [3, 12], [0, 0]),
]


@pytest.mark.parametrize("name,hq,hkv,ctx,ql,draft", TAIL_CASES, ids=[c[0] for c in TAIL_CASES])
def test_stale_tail_slots_are_masked(gpu, name, hq, hkv, ctx, ql, draft):
    """Slots past kv_len on a row's current page may hold anything (here NaN keys and +inf
    values): the output stays finite and equals the oracle, which reads only kv_len keys."""
    say("tail masking", name)
    step = build_step(hq=hq, hkv=hkv, ctx_len=ctx, q_len=ql, is_draft=draft, draft_budget=12, seed=31, device=gpu)
    cache = step.cache.clone()
    assert _poison_tails(cache, step) == len(ctx)
    w = make_wrapper(gpu)
    plan(w, step)
    out, lse = w.run(step.q, cache, return_lse=True)
    torch.cuda.synchronize()
    T = step.total_tokens
    ref_out, ref_lse = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                                       step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=hkv)
    attn_close(out[:T], ref_out[:T])
    assert (lse[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3


def test_stale_tail_slots_masked_for_per_head_lists_scores_and_dump(gpu):
    """The same poisoned tails under a segment plan (verify rows staged over a shared list,
    draft rows direct over one list per head), and under the refresh epilogues: key-mean page
    scores and the first/last dump never read or write past kv_len."""
    say("tail masking: per-head lists, scores, dump")
    hq, hkv = 32, 8
    ctx = np.array([1 + 16 * 70, 9 + 16 * 30, 14 + 16 * 12, 4 + 16 * 55])
    ql = np.array([1, 4, 1, 9])
    step = build_step(hq=hq, hkv=hkv, ctx_len=ctx, q_len=ql, is_draft=[0] * 4, draft_budget=0, seed=32, device=gpu)
    cache = step.cache.clone()
    _poison_tails(cache, step)
    table = step.block_table.cpu().numpy()
    n_pages = (ctx + 15) // 16
    last = (ctx - 1) % 16 + 1
    rng = np.random.default_rng(3)
    idx, start, pages, kvl = [], [], [], []
    pos = 0
    for b in range(len(ctx)):
        n = int(n_pages[b])
        if ql[b] == 1:
            for g in range(hkv):
                k = min(20, n)
                sel = np.sort(np.concatenate([rng.choice(n - 1, size=k - 1, replace=False), [n - 1]]))
                idx.append(table[b, sel])
                start.append(pos)
                pos += k
                pages.append(k)
                kvl.append((k - 1) * 16 + int(last[b]))
        else:
            idx.append(table[b, :n])
            start += [pos] * hkv
            pages += [n] * hkv
            kvl += [int(ctx[b])] * hkv
            pos += n
    flat = np.concatenate(idx).astype(np.int32)
    w = make_wrapper(gpu)
    plan(w, step)
    t32 = lambda a: torch.tensor(np.asarray(a), dtype=torch.int32)
    w.plan_segments(step.qo_indptr_host[: len(ctx) + 1], t32(start), t32(pages), t32(kvl),
                    torch.from_numpy(flat).to(gpu), hq, hkv, 128, PAGE, causal=True)
    out, lse = w.run(step.q, cache, return_lse=True)
    torch.cuda.synchronize()
    kvp_o = np.concatenate([[0], np.cumsum(pages)])
    idx_o = np.concatenate([flat[s0 : s0 + n] for s0, n in zip(start, pages)])
    ref_out, ref_lse = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host[: len(ctx) + 1], kvp_o,
                                       torch.from_numpy(idx_o), kvl, num_kv_heads=hkv, per_head_lists=True)
    T = int(ql.sum())
    attn_close(out[:T], ref_out[:T])
    assert (lse[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3

    # refresh epilogues over the poisoned cache: full row lists, page scores and the dump
    args = build_holistic_dump_jit_args(torch.bfloat16, 128, dump_kind="first_last_compact",
                                        dump_buffer_dtype=torch.float16)
    wd = make_wrapper(gpu, jit_args=args)
    plan(wd, step)
    stride = int(n_pages.max()) * 16
    dump = torch.full((len(ctx) * hq * 2 * stride,), float("-inf"), dtype=torch.float16, device=gpu)
    ps = torch.full((len(ctx) * hkv, int(n_pages.max())), float("nan"), device=gpu)
    out_d, _ = wd.run(step.q, cache, dump, hq, stride, return_lse=True, page_scores=ps)
    torch.cuda.synchronize()
    ref_dump = torch.full((len(ctx) * hq * 2 * stride,), float("-inf"), dtype=torch.float16)
    ref_ps = torch.full((len(ctx) * hkv, int(n_pages.max())), float("nan"))
    ref_out_d, _ = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                                   step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=hkv, page_scores=ref_ps,
                                   dump=DumpSpec(buffer=ref_dump, kind="first_last", num_heads=hq, kv_stride=stride))
    attn_close(out_d[:T], ref_out_d[:T])
    got, ref = dump.cpu().float(), ref_dump.float()
    written = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), written)
    assert torch.allclose(got[written], ref[written], rtol=2e-3, atol=2e-3)
    fin = ~torch.isnan(ref_ps)
    assert torch.equal(~torch.isnan(ps.cpu()), fin)
    assert torch.allclose(ps.cpu()[fin], ref_ps[fin], rtol=1e-4, atol=1e-4)
