"""BASELINE config 3 at its real workload: the full 36-layer Qwen3-8B decode step, batch 64,
contexts U[8192, 32768], a 50/50 draft/verify mix with verify q_len U{2..9}, refresh at layer 2
with the top-128 pages per (row, KV head).

The step runs once eagerly with every layer's intermediates captured. Checks:
* the logits are finite and the token ids are their first-index argmax;
* the draft rows' selection is the exact top-128 (current page forced in) of the GPU's own
  key-mean scores, for all 32 draft rows x 8 kv heads;
* in the refresh layer and in two mixed layers, q after the fused q/k RMSNorm + RoPE equals
  the oracle on the captured projections (one bf16 rounding), every appended K/V row is in its
  page slot (V bit-exact), and the attention output of 2 draft and 2 verify rows (one with
  q_len 9) equals the oracle over the row's page lists;
* the step recorded in one HIP graph replays to the eager ids and logits.
The model is ~16 GB of weights and ~186 GB of KV pages; everything is freed at the end.
"""

import numpy as np
import pytest
import torch

from aspire_amd.decode_step import QWEN3_8B, DecodeWeights, MixedDecodeStep, alloc_kv_caches
from aspire_amd.workloads import PAGE, config3_rows, random_block_table
from helpers import attn_close, bits, oracle_row, say
from oracle import decode as odecode
from oracle.rope import qk_norm_rope
from oracle.select import topk_pages_per_head

pytestmark = pytest.mark.gpu

CHECK_LAYERS = (2, 20, 35)   # the refresh layer and two mixed layers


def rotated_close(got: torch.Tensor, ref: torch.Tensor, what: str):
    """Rotated q/k within two bf16 rounding steps of the reference, measured against the norm of
    each rotated pair (dims 2i, 2i+1). The RMSNorm rounds twice (x * rsqrt, then * weight), and
    its fp32 sum order can move either rounding by a step; the rotation keeps the pair's norm and
    spreads an input's error over both outputs of the pair, however small the output itself
    (a*cos - b*sin can cancel)."""
    g, r = got.float().cpu(), ref.float().cpu()
    pair = torch.sqrt(r[..., 0::2] ** 2 + r[..., 1::2] ** 2).repeat_interleave(2, dim=-1)
    err = (g - r).abs() / (pair + 1e-6)
    bad = err > 2.0 ** -6
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} values off, worst {float(err.max()):.4g}"
    assert float(err.mean()) < 2.0 ** -9, f"{what}: mean error {float(err.mean()):.4g} of the pair norm"


def test_config3_full_decode_step(gpu):
    say("config3: 36-layer Qwen3-8B step, B=64")
    torch.cuda.empty_cache()
    shape = QWEN3_8B
    ctx, ql, dr = config3_rows(seed=0)
    n_pages = (ctx + PAGE - 1) // PAGE
    table, pool = random_block_table(n_pages, seed=0)
    weights = DecodeWeights(shape, gpu, seed=0)
    caches = alloc_kv_caches(shape, pool, gpu, seed=0)
    step = MixedDecodeStep(weights, caches, ctx, ql, dr, torch.from_numpy(table), budget=128, refresh_layer=2)
    try:
        _check(step, shape, ctx, ql, dr, table, gpu)
    finally:
        del step, caches, weights
        torch.cuda.empty_cache()


def _check(step, shape, ctx, ql, dr, table, gpu):
    B, H, T = step.batch, step.heads, step.T
    assert B == 64 and T == int(ql.sum()) and 9 in ql[~dr].tolist()
    state = [step.selector.selected, step.selector.counts, step.mixed_indices, step.mixed_indptr]
    saved = [t.clone() for t in state]
    cap = {}
    say("config3: eager step")
    ids = step.forward(capture=cap).clone()
    logits = step.logits.clone()
    torch.cuda.synchronize()
    assert torch.isfinite(logits.float()).all()
    assert torch.equal(ids.cpu(), odecode.argmax_rows(logits.cpu()))

    # selection: exact top-128 of the GPU's key-mean scores, the current page forced in
    say("config3: selection")
    scores = step.selector.page_scores[: B * H].cpu()
    sel = step.selector.selected[:B].cpu().numpy()
    cnt = step.selector.counts[:B].cpu().numpy()
    n_pages = (ctx + PAGE - 1) // PAGE
    logical, c = topk_pages_per_head(scores, np.repeat(n_pages, H), 128, 1)
    logical = logical.numpy().reshape(B, H, -1)
    for b in np.flatnonzero(dr):
        for g in range(H):
            k = int(c[b * H + g])
            assert cnt[b, g] == k == min(128, int(n_pages[b]))
            assert sel[b, g, :k].tolist() == table[b][logical[b, g, :k]].tolist(), (b, g)

    # per-layer parity on sampled rows
    drafts = np.flatnonzero(dr)
    verify = np.flatnonzero(~dr)
    v9 = int(verify[np.flatnonzero(ql[verify] == 9)[0]])
    v_other = int(verify[np.argmin(ql[verify])])
    rows = [int(drafts[0]), int(drafts[-1]), v9, v_other]
    qo = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
    offsets = (ctx - ql).astype(np.int32)
    qs, kvs = shape.q_size, shape.kv_size
    tok_row = np.repeat(np.arange(B), ql)
    tok_pos = np.concatenate([np.arange(ctx[b] - ql[b], ctx[b]) for b in range(B)])
    tok_page = torch.from_numpy(table[tok_row, tok_pos // PAGE].astype(np.int64)).to(gpu)
    tok_slot = torch.from_numpy((tok_pos % PAGE).astype(np.int64)).to(gpu)
    seg_start = step.seg_start_host.numpy()
    seg_pages = step.seg_pages_host.numpy()
    seg_len = step.mixed_kv_len_host.numpy()
    mixed_idx = step.mixed_indices.cpu().numpy()
    for layer in CHECK_LAYERS:
        say(f"config3: layer {layer}")
        lw = step.w.layers[layer]
        qkv = cap[f"qkv{layer}"].cpu()
        q_raw = qkv[:, :qs].reshape(T, shape.n_head, shape.head_dim)
        k_raw = qkv[:, qs : qs + kvs].reshape(T, shape.n_local_heads, shape.head_dim)
        v_raw = qkv[:, qs + kvs :].reshape(T, shape.n_local_heads, shape.head_dim)
        ref_q, ref_k = qk_norm_rope(q_raw, k_raw, qo, offsets, theta=shape.rope_base, q_weight=lw["q_norm"].cpu(),
                                    k_weight=lw["k_norm"].cpu(), eps=shape.norm_eps)
        rotated_close(cap[f"q{layer}"], ref_q, f"layer {layer} q")
        # the appended rows sit in their page slots: rotated k within a rounding, v exact
        kv_new = step.caches[layer][tok_page, :, tok_slot].cpu()   # [T, 2, H_kv, 128]
        rotated_close(kv_new[:, 0], ref_k, f"layer {layer} appended k")
        assert (bits(kv_new[:, 1]) == bits(v_raw)).all(), f"layer {layer} appended v"
        y = cap[f"y{layer}"]
        for b in rows:
            toks = range(int(qo[b]), int(qo[b + 1]))
            if layer == step.refresh_layer or not dr[b]:
                pages, lens, per_head = table[b, : n_pages[b]], [int(ctx[b])], False
            else:
                segs = range(b * H, (b + 1) * H)
                pages = [mixed_idx[seg_start[s] : seg_start[s] + seg_pages[s]] for s in segs]
                lens = [int(seg_len[s]) for s in segs]
                per_head = True
                for g, s in enumerate(segs):   # a draft head's list is its selection
                    assert pages[g].tolist() == sel[b, g, : cnt[b, g]].tolist()
            ref_out, _ = oracle_row(cap[f"q{layer}"], step.caches[layer], toks, pages, lens, shape.n_local_heads,
                                    per_head=per_head)
            attn_close(y[list(toks)], ref_out)
    del cap

    # graph replay from the same state equals the eager step
    say("config3: graph replay")
    for t, s in zip(state, saved):
        t.copy_(s)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step.forward()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gids = step.forward()
    glogits = step.logits
    for rep in range(2):
        for t, s in zip(state, saved):
            t.copy_(s)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gids, ids), f"replay {rep} ids"
        assert torch.equal(glogits, logits), f"replay {rep} logits"
        _ = torch.randn(1000, device=gpu).sum().item()   # eager work between replays
    del graph


def test_config3_first_last_refresh(gpu):
    """The reference's own refresh inside the config-3 step (selector="first_last"): the refresh
    layer writes the fp16 first/last logits dump and the LSE of every row; the next step's
    preparation selects each row's top-128 pages with PageSelectorFirstLastAvg (last 8 forced in)
    and builds one list per row with build_unified_indices, which the mixed layers attend. Checks:
    * page scores equal the oracle's restatement of page_selector.py on the GPU's own dump and
      LSE, and the selected sets are exact wherever the score gap exceeds 1e-3 (all 64 rows);
    * the refresh layer's dump of sampled rows equals fp16(q.k) of the oracle (one fp16 step);
    * in the refresh layer and two mixed layers, 2 draft rows (over their selection) and 2 verify
      rows (one with q_len 9, over the full table) equal the oracle;
    * the step recorded in one HIP graph (selection included) replays to the eager ids and logits.
    """
    from oracle.attention import DumpSpec
    from oracle.select import FirstLastSelector
    from helpers import assert_topk_sets

    say("config3 (R): 36-layer Qwen3-8B step, B=64, first/last refresh")
    torch.cuda.empty_cache()
    shape = QWEN3_8B
    ctx, ql, dr = config3_rows(seed=0)
    n_pages = (ctx + PAGE - 1) // PAGE
    table, pool = random_block_table(n_pages, seed=0)
    weights = DecodeWeights(shape, gpu, seed=0)
    caches = alloc_kv_caches(shape, pool, gpu, seed=0)
    step = MixedDecodeStep(weights, caches, ctx, ql, dr, torch.from_numpy(table), budget=128, refresh_layer=2,
                           selector="first_last")
    try:
        B, T, Hq = step.batch, step.T, shape.n_head
        W, stride = table.shape[1], step.kv_stride
        say("config3 (R): step 1")
        step.forward()
        torch.cuda.synchronize()
        dump, lse = step.dump.cpu(), step.lse_buf.cpu()
        qo = np.concatenate([[0], np.cumsum(ql)]).astype(np.int32)
        say("config3 (R): selection")
        step.select_first_last()
        torch.cuda.synchronize()
        sel = step.fl_selected.cpu().numpy()
        valid = step.fl_valid.cpu().numpy()
        got_scores = step.fl_selector._scores[:B].cpu().numpy()
        ref = FirstLastSelector(pages_per_slot=W, subset_cache_size=128, L=8, n_heads=Hq, page_size=PAGE,
                                max_seq_length=W * PAGE, bsz=B, kv_stride=stride)
        ref_scores = ref.page_scores(dump, lse, torch.from_numpy(qo))
        eff = ref.effective_scores(ref_scores, torch.from_numpy(n_pages.astype(np.int32))).double().numpy()
        ref_scores = ref_scores.numpy()
        for b in range(B):
            n = int(n_pages[b])
            assert np.allclose(got_scores[b, :n], ref_scores[b, :n], rtol=1e-5, atol=1e-6), b
            k = int(valid[b])
            assert k == min(128, n)
            inv = {int(p): j for j, p in enumerate(table[b, :n])}
            logical = [inv[int(p)] for p in sel[b, :k]]
            assert logical == sorted(logical) and logical[-1] == n - 1, b
            assert_topk_sets(logical, eff[b, :n], k)
        del ref_scores, eff

        say("config3 (R): step 2 with the selection")
        state = [step.dump, step.lse_buf]
        saved = [t.clone() for t in state]
        cap = {}
        ids = step.forward(capture=cap).clone()
        logits = step.logits.clone()
        torch.cuda.synchronize()
        assert torch.isfinite(logits.float()).all()
        row_ptr = step.row_indptr.cpu().numpy()
        row_idx = step.row_indices.cpu().numpy()
        drafts, verify = np.flatnonzero(dr), np.flatnonzero(~dr)
        v9 = int(verify[np.flatnonzero(ql[verify] == 9)[0]])
        rows = [int(drafts[0]), int(drafts[-1]), v9, int(verify[np.argmin(ql[verify])])]
        dump2 = step.dump.view(B, Hq, 2, stride)
        for layer in (2, 20, 35):
            say(f"config3 (R): layer {layer}")
            y = cap[f"y{layer}"]
            for b in rows:
                toks = range(int(qo[b]), int(qo[b + 1]))
                if layer == step.refresh_layer or not dr[b]:
                    pages, lens = table[b, : n_pages[b]], [int(ctx[b])]
                else:
                    pages = row_idx[row_ptr[b] : row_ptr[b + 1]]
                    assert pages.tolist() == sel[b, : valid[b]].tolist()
                    lens = [int(valid[b] - 1) * PAGE + (int(ctx[b]) - 1) % PAGE + 1]
                kw = {}
                if layer == step.refresh_layer:
                    ref_dump = torch.full((Hq * 2 * stride,), float("-inf"), dtype=torch.float16)
                    kw["dump"] = DumpSpec(buffer=ref_dump, kind="first_last", num_heads=Hq, kv_stride=stride)
                ref_out, _ = oracle_row(cap[f"q{layer}"], step.caches[layer], toks, pages, lens, shape.n_local_heads,
                                        **kw)
                attn_close(y[list(toks)], ref_out)
                if layer == step.refresh_layer:
                    got = dump2[b].cpu().float().reshape(-1)
                    want = ref_dump.float()
                    written = torch.isfinite(want)
                    slots = 2 if ql[b] > 1 else 1
                    # the row's written entries (slot 1 of a single-query row keeps its earlier values)
                    mask = written.view(Hq, 2, stride)[:, :slots].reshape(-1)
                    g2 = got.view(Hq, 2, stride)[:, :slots].reshape(-1)
                    w2 = want.view(Hq, 2, stride)[:, :slots].reshape(-1)
                    assert torch.equal(torch.isfinite(g2), mask), b
                    assert torch.allclose(g2[mask], w2[mask], rtol=2e-3, atol=2e-3), b
        del cap

        say("config3 (R): graph replay")
        for t, s_ in zip(state, saved):
            t.copy_(s_)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step.forward()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            gids = step.forward()
        glogits = step.logits
        for rep in range(2):
            for t, s_ in zip(state, saved):
                t.copy_(s_)
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(gids, ids), f"replay {rep} ids"
            assert torch.equal(glogits, logits), f"replay {rep} logits"
            _ = torch.randn(1000, device=gpu).sum().item()
        del graph
    finally:
        del step, caches, weights
        torch.cuda.empty_cache()
