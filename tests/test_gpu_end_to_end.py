"""Config 0 end to end, as a refresh step runs it in the reference (base.py:516-541, 580-667,
1128-1376): the refresh layer attends every row's full context and writes the first/last
logits dump; the (R) selector turns the dump into each draft row's top-64 pages; the
mixed page list is built from those selections; the mixed draft/verify layer runs over it.
Every stage is checked against the CPU oracle on the stage's own inputs."""

import numpy as np
import pytest
import torch

from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper, build_holistic_dump_jit_args
from aspire_amd.attention.page_list import build_unified_indices
from aspire_amd.backends.page_selector import PageSelectorFirstLastAvg
from aspire_amd.workloads import PAGE, build_step, config0
from helpers import assert_topk_sets, attn_close, say
from oracle.attention import DumpSpec, paged_attention
from oracle.page_list import build_unified_indices as oracle_unified_indices
from oracle.select import FirstLastSelector

pytestmark = pytest.mark.gpu


def test_config0_refresh_select_then_mixed_step(gpu):
    say("config0 end to end")
    base = config0(device=gpu)  # rows 0-1 draft (q_len 1), rows 2-3 verify (q_len 5); 4096 tokens each
    B, H, HKV = base.batch, base.hq, base.hkv
    pages = int(base.block_table.shape[1])
    ctx = int(base.ctx_len[0])
    assert pages * PAGE == ctx and (base.ctx_len == ctx).all()
    T = base.total_tokens
    table = base.block_table
    qo_host = base.qo_indptr_host

    # --- refresh layer: full context for every row, first/last fp16 dump ------------------
    full_ptr = torch.tensor([0] + [pages * (b + 1) for b in range(B)] + [pages * B], dtype=torch.int32)
    full_idx = table.reshape(-1).contiguous()
    full_last = torch.tensor([PAGE] * B + [0], dtype=torch.int32, device=gpu)
    full_len = torch.tensor([ctx] * B + [0], dtype=torch.int32)
    kv_stride = ctx
    args = build_holistic_dump_jit_args(torch.bfloat16, 128, dump_kind="first_last_compact",
                                        dump_buffer_dtype=torch.float16)
    wr = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD", jit_args=args)
    wr.plan(base.qo_indptr, full_ptr.to(gpu), full_idx, full_last, H, HKV, 128, PAGE, causal=True)
    dump = torch.full((B * H * 2 * kv_stride,), float("-inf"), dtype=torch.float16, device=gpu)
    out_r, lse_r = wr.run(base.q, base.cache, dump, H, kv_stride, return_lse=True)
    torch.cuda.synchronize()
    ref_dump = torch.full((B * H * 2 * kv_stride,), float("-inf"), dtype=torch.float16)
    ref_out, ref_lse = paged_attention(base.q.cpu(), base.cache.cpu(), qo_host, full_ptr, full_idx.cpu(), full_len,
                                       num_kv_heads=HKV, dump=DumpSpec(buffer=ref_dump, kind="first_last",
                                                                       num_heads=H, kv_stride=kv_stride))
    attn_close(out_r[:T], ref_out[:T])
    assert (lse_r[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3
    got, ref = dump.cpu().float(), ref_dump.float()
    written = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), written)
    assert torch.allclose(got[written], ref[written], rtol=2e-3, atol=2e-3)

    # --- (R) selector over the GPU dump: top-64 pages per row, the last page forced in ------
    kw = dict(pages_per_slot=pages, subset_cache_size=64, L=1, n_heads=H, page_size=PAGE, max_seq_length=ctx,
              bsz=B, head_dim=128, kv_stride=kv_stride, draft_percent=None, min_draft_pages=None)
    sel = PageSelectorFirstLastAvg(max_batch_size=B, device=gpu, dec_len=8, **kw)
    npg = torch.full((B,), pages, dtype=torch.int32, device=gpu)
    selected, valid = sel.select(dump, lse_r[:T].contiguous(), npg, table, base.qo_indptr)
    selected, valid = selected.clone(), valid.clone()
    torch.cuda.synchronize()
    osel = FirstLastSelector(**kw)
    scores = osel.page_scores(dump.cpu(), lse_r[:T].cpu(), qo_host)
    eff = osel.effective_scores(scores, npg.cpu())
    tab = table.cpu().numpy()
    assert valid.tolist() == [64] * B
    for b in range(B):
        inv = {int(p): j for j, p in enumerate(tab[b])}
        logical = [inv[int(p)] for p in selected[b].cpu().numpy()]
        # default (logical) order: ascending logical pages, so the current page, forced in by L = 1,
        # is the list's last entry, as the mixed layer's kv_len assumes (the reference's physical
        # order gives the same list on its arange block table; this table is a random permutation)
        assert np.all(np.diff(logical) > 0) and logical[-1] == pages - 1
        assert_topk_sets(logical, eff[b].double().numpy(), 64)

    # --- mixed page list: draft rows 0-1 use their selections, verify rows 2-3 the full table -
    mode = base.mode_flags
    dn = valid.clone()
    vn = torch.full((B,), pages, dtype=torch.int32, device=gpu)
    idx = torch.zeros(B * pages, dtype=torch.int32, device=gpu)
    ptr = torch.zeros(B + 2, dtype=torch.int32, device=gpu)
    build_unified_indices(mode, selected, table, dn, vn, idx, ptr, indptr_fill_to=B + 2)
    torch.cuda.synchronize()
    ref_idx = np.zeros(B * pages, dtype=np.int32)
    ref_ptr = np.zeros(B + 2, dtype=np.int32)
    oracle_unified_indices(mode.cpu().numpy(), selected.cpu().numpy(), tab, dn.cpu().numpy(), vn.cpu().numpy(),
                           ref_idx, ref_ptr)
    ref_ptr[B + 1] = ref_ptr[B]
    n_entries = int(ref_ptr[B])
    assert ptr.cpu().numpy().tolist() == ref_ptr.tolist()
    assert np.array_equal(idx[:n_entries].cpu().numpy(), ref_idx[:n_entries])

    # --- the mixed draft/verify layer over those lists ---------------------------------------
    lists = ref_ptr[1 : B + 1] - ref_ptr[:B]
    kv_len = torch.tensor(list((lists - 1) * PAGE + PAGE) + [0], dtype=torch.int32)
    wm = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD")
    wm.plan(base.qo_indptr, ptr, idx, full_last, H, HKV, 128, PAGE, causal=True)
    out_m, lse_m = wm.run(base.q, base.cache, return_lse=True)
    torch.cuda.synchronize()
    ref_out_m, ref_lse_m = paged_attention(base.q.cpu(), base.cache.cpu(), qo_host, torch.from_numpy(ref_ptr),
                                           torch.from_numpy(ref_idx), kv_len, num_kv_heads=HKV)
    attn_close(out_m[:T], ref_out_m[:T])
    assert (lse_m[:T].cpu() - ref_lse_m[:T]).abs().max() < 2e-3
    # the draft rows now attend 64 of their 256 pages: their output differs from the refresh layer's
    assert (out_m[:2].float() - out_r[:2].float()).abs().max() > 1e-3


def test_stale_slot1_survives_a_draft_step(gpu):
    """Two refresh steps on one dump buffer, as the reference runs them: the buffer is filled
    with -inf once (base.py:324-330) and only cleared per slot on refill (base.py:1404-1419).
    Step 1: rows 0-2 verify (their first and last queries dump slots 0 and 1), row 3 drafts.
    Step 2: rows 0, 1 and 3 draft (a single query dumps slot 0 only), row 2 verifies again. The
    slot-1 logits of rows 0 and 1 are step 1's, and the selector re-normalises them with the
    step-2 LSE (page_selector.py:206-214); GPU and oracle carry the same state."""
    say("stale slot 1 across two steps")
    H, HKV = 16, 8
    ctx = [600, 900, 450, 1000]
    kw = dict(hq=H, hkv=HKV, ctx_len=ctx, is_draft=[0] * 4, draft_budget=0, seed=31, device=gpu)
    s1 = build_step(q_len=[5, 3, 4, 1], **kw)
    s2 = build_step(q_len=[1, 1, 2, 1], **kw)      # same seed and lengths: the same cache and table
    assert torch.equal(s1.cache, s2.cache) and torch.equal(s1.block_table, s2.block_table)
    B = 4
    stride = 1024
    args = build_holistic_dump_jit_args(torch.bfloat16, 128, dump_kind="first_last_compact",
                                        dump_buffer_dtype=torch.float16)
    w = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD", jit_args=args)
    dump = torch.full((B * H * 2 * stride,), float("-inf"), dtype=torch.float16, device=gpu)
    ref_dump = torch.full((B * H * 2 * stride,), float("-inf"), dtype=torch.float16)
    pages = int(s1.block_table.shape[1])
    kw_sel = dict(pages_per_slot=pages, subset_cache_size=12, L=2, n_heads=H, page_size=PAGE,
                  max_seq_length=pages * PAGE, bsz=B, head_dim=128, kv_stride=stride, draft_percent=None,
                  min_draft_pages=None)
    sel = PageSelectorFirstLastAvg(max_batch_size=B, device=gpu, dec_len=8, **kw_sel)
    osel = FirstLastSelector(**kw_sel)
    npg = torch.tensor([(c + 15) // 16 for c in ctx], dtype=torch.int32, device=gpu)
    view = dump.view(B, H, 2, stride)
    for i, st in enumerate((s1, s2)):
        w.plan(st.qo_indptr, st.kv_indptr, st.kv_indices, st.last_page_len, H, HKV, 128, PAGE, causal=True)
        before = view.clone()
        _, lse = w.run(st.q, st.cache, dump, H, stride, return_lse=True)
        T = st.total_tokens
        selected, valid = sel.select(dump, lse[:T].contiguous(), npg, st.block_table, st.qo_indptr)
        torch.cuda.synchronize()
        paged_attention(st.q.cpu(), st.cache.cpu(), st.qo_indptr_host, st.kv_indptr_host, st.kv_indices.cpu(),
                        st.kv_len_host, num_kv_heads=HKV,
                        dump=DumpSpec(buffer=ref_dump, kind="first_last", num_heads=H, kv_stride=stride))
        got, ref = dump.cpu().float(), ref_dump.float()
        written = torch.isfinite(ref)
        assert torch.equal(torch.isfinite(got), written), f"step {i + 1}: dump entries"
        assert torch.allclose(got[written], ref[written], rtol=2e-3, atol=2e-3), f"step {i + 1}"
        if i == 1:
            # single-query rows 0, 1, 3 left slot 1 as step 1 wrote it, bit for bit
            for b in (0, 1, 3):
                assert torch.equal(view[b, :, 1], before[b, :, 1]), b
            assert torch.isfinite(view[0, :, 1, : ctx[0]]).all()   # stale but present (row 0 verified)
            assert torch.isinf(view[3, :, 1]).all()                  # row 3 never verified
        # the selection over the carried buffer (GPU dump, GPU LSE) against the oracle chain
        scores = osel.page_scores(dump.cpu(), lse[:T].cpu(), st.qo_indptr_host)
        eff = osel.effective_scores(scores, npg.cpu())
        ref_sel, ref_valid = osel.finalize(scores, npg.cpu(), st.block_table.cpu(), order="logical")
        assert torch.equal(valid.cpu(), ref_valid)
        tab = st.block_table.cpu().numpy()
        for b in range(B):
            k = int(valid[b])
            # rows shorter than the table are zero-padded: map only the row's own pages
            inv = {int(p): j for j, p in enumerate(tab[b, : int(npg[b])])}
            logical = [inv[int(p)] for p in selected[b, :k].cpu().numpy()]
            assert_topk_sets(logical, eff[b].double().numpy(), k)
        if i == 1:
            # the stale slot matters: clearing it changes row 0's scores
            cleared = dump.cpu().clone().view(B, H, 2, stride)
            cleared[0, :, 1] = float("-inf")
            s_clear = osel.page_scores(cleared.view(-1), lse[:T].cpu(), st.qo_indptr_host)
            assert (s_clear[0] - scores[0]).abs().max() > 1e-3
