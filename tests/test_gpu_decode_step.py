"""The full decode step's GPU pieces against the CPU oracle: the row kernels, the per-head
page lists, a small model step end to end, and the step recorded in a HIP graph."""

import numpy as np
import pytest
import torch

from aspire_amd.attention.page_list import build_head_page_lists
from aspire_amd.decode_step import (DecodeWeights, MixedDecodeStep, ModelShape, add_rms_norm, alloc_kv_caches,
                                    argmax_rows, silu_mul)
from aspire_amd.workloads import random_block_table
from helpers import bits, say
from oracle import decode as odecode
from oracle.page_list import build_head_page_lists as oracle_head_lists
from oracle.select import topk_pages_per_head

pytestmark = pytest.mark.gpu


def ulp_diff(a: torch.Tensor, b: torch.Tensor) -> int:
    """Largest distance in bf16 steps between two bf16 tensors of the same sign pattern."""
    x = bits(a).astype(np.int32)
    y = bits(b).astype(np.int32)
    x = np.where(x & 0x8000, -(x & 0x7FFF), x)
    y = np.where(y & 0x8000, -(y & 0x7FFF), y)
    return int(np.abs(x - y).max()) if x.size else 0


@pytest.mark.parametrize("dim,rows", [(4096, 37), (512, 5), (8192, 3)])
def test_add_rms_norm(gpu, dim, rows):
    say("add_rms_norm", dim, rows)
    g = torch.Generator().manual_seed(dim)
    x = (torch.randn(rows, dim, generator=g) * 3).to(torch.bfloat16)
    d = torch.randn(rows, dim, generator=g).to(torch.bfloat16)
    w = (torch.rand(dim, generator=g) + 0.5).to(torch.bfloat16)
    xg, dg, wg = x.to(gpu), d.to(gpu), w.to(gpu)
    out = torch.empty_like(xg)
    add_rms_norm(xg, wg, out, 1e-6, delta=dg)
    x2, ref = odecode.add_rms_norm(x, w, 1e-6, d)
    assert torch.equal(xg.cpu(), x2)                      # the residual add is exact
    assert ulp_diff(out.cpu(), ref) <= 1                  # the fp32 sum order only moves a rounding
    out2 = torch.empty_like(xg)
    add_rms_norm(xg, wg, out2, 1e-6)                      # no delta: x is left as it is
    assert torch.equal(xg.cpu(), x2) and torch.equal(out2, out)


@pytest.mark.parametrize("inter,rows", [(12288, 9), (1024, 3)])
def test_silu_mul(gpu, inter, rows):
    say("silu_mul", inter, rows)
    g = torch.Generator().manual_seed(inter)
    gu = (torch.randn(rows, 2 * inter, generator=g) * 4).to(torch.bfloat16)
    out = torch.empty(rows, inter, dtype=torch.bfloat16, device=gpu)
    silu_mul(gu.to(gpu), out)
    ref = odecode.silu_mul(gu)
    assert ulp_diff(out.cpu(), ref) <= 1
    assert (bits(out.cpu()) == bits(ref)).mean() > 0.99


def test_argmax_rows(gpu):
    say("argmax_rows")
    g = torch.Generator().manual_seed(1)
    vocab, stride = 1003, 1008                           # a tail past the last 8-wide chunk
    x = torch.randn(6, stride, generator=g).to(torch.bfloat16)
    x[0, 5] = x[0, 900] = 9.0                            # tie: the first index wins
    x[1, 1002] = 9.0                                     # the maximum in the tail
    x[2, :] = float("-inf")
    x[3, 1003:] = 50.0                                   # beyond vocab: never looked at
    ids = torch.zeros(6, dtype=torch.int64, device=gpu)
    argmax_rows(x.to(gpu)[:, :vocab], ids)
    ref = odecode.argmax_rows(x[:, :vocab])
    assert ids.cpu().tolist() == ref.tolist()
    assert ids[0].item() == 5 and ids[1].item() == 1002 and ids[2].item() == 0
    big = torch.randn(208, 151936, generator=g).to(torch.bfloat16)
    ids = torch.zeros(208, dtype=torch.int64, device=gpu)
    argmax_rows(big.to(gpu), ids)
    assert torch.equal(ids.cpu(), odecode.argmax_rows(big))


@pytest.mark.parametrize("share", [False, True])
def test_head_page_lists(gpu, share):
    say("head page lists", share)
    rng = np.random.default_rng(4)
    B, H, K, W = 13, 8, 128, 900
    mode = rng.integers(0, 2, B).astype(np.int32)
    vn = rng.integers(0, W + 1, B).astype(np.int32)
    table = rng.integers(0, 1 << 20, (B, W)).astype(np.int32)
    sel = rng.integers(0, 1 << 20, (B, H, K)).astype(np.int32)
    cnt = rng.integers(0, K + 1, (B, H)).astype(np.int32)
    cap = B * H * W
    idx = torch.full((cap,), -1, dtype=torch.int32, device=gpu)
    ptr = torch.full((B * H + 3,), -1, dtype=torch.int32, device=gpu)
    t = lambda a: torch.from_numpy(a).to(gpu)
    build_head_page_lists(t(mode), t(sel), t(cnt), t(table), t(vn), idx, ptr, share_verify=share,
                          indptr_fill_to=B * H + 3)
    torch.cuda.synchronize()
    ref_idx = np.full(cap, -1, dtype=np.int64)
    ref_ptr = np.zeros(B * H + 1, dtype=np.int64)
    oracle_head_lists(mode, sel, cnt, table, vn, ref_idx, ref_ptr, share_verify=share)
    got_ptr = ptr.cpu().numpy()
    assert np.array_equal(got_ptr[: B * H + 1], ref_ptr)
    assert (got_ptr[B * H + 1 :] == ref_ptr[-1]).all()
    n = int(ref_ptr[-1])
    assert np.array_equal(idx[:n].cpu().numpy(), ref_idx[:n]) and (idx[n:].cpu() == -1).all()


SMALL = ModelShape(n_layer=4, dim=512, n_head=8, n_local_heads=2, head_dim=128, intermediate_size=1024,
                   vocab_size=1024, rope_base=1e6)
# Qwen3-8B's attention shape (32 q / 8 kv heads, GQA 4) on a small model: 8 kv heads per slot put the
# verify rows' shared lists on the staged LDS path, with the draft rows' per-head lists direct, in one
# launch (the mix the full decode step runs)
SMALL_GQA4 = ModelShape(n_layer=4, dim=512, n_head=32, n_local_heads=8, head_dim=128, intermediate_size=1024,
                        vocab_size=1024, rope_base=1e6)
SHAPES = [pytest.param(SMALL, id="gqa4_hkv2"), pytest.param(SMALL_GQA4, id="gqa4_hkv8")]


def _small_step(gpu, budget=8, seed=0, shape=SMALL):
    ctx = np.array([700, 1500, 333, 1200, 260, 980])
    ql = np.array([1, 2, 1, 5, 1, 9])                  # verify rows fill 8, 20 and 36 query rows
    dr = ql == 1
    n_pages = (ctx + 15) // 16
    table, pool = random_block_table(n_pages, seed=seed, pool_pages=int(n_pages.sum()) + 11)
    w = DecodeWeights(shape, gpu, seed=seed)
    caches = alloc_kv_caches(shape, pool, gpu, seed=seed)
    step = MixedDecodeStep(w, caches, ctx, ql, dr, torch.from_numpy(table), budget=budget, refresh_layer=2)
    return step, ctx, ql, dr, table


@pytest.mark.parametrize("shape", SHAPES)
def test_small_decode_step_matches_oracle(gpu, shape):
    say("small decode step", shape)
    step, ctx, ql, dr, table = _small_step(gpu, shape=shape)
    B, H = step.batch, step.heads
    init_sel = step.selector.selected.cpu().numpy().copy()
    init_cnt = step.selector.counts.cpu().numpy().copy()
    caches0 = step.caches.cpu()
    cap = {}
    ids = step.forward(capture=cap)
    torch.cuda.synchronize()
    # the mixed layers ran one head-aligned plan: a slot is the row's n_local_heads waves
    # (int 4 of the plan header), so with 8 kv heads the verify rows stage their shared pages
    hpu = int(step.mixed_wrapper._int_workspace[16:20].view(torch.int32).item())
    assert hpu == shape.n_local_heads
    sel = step.selector.selected.cpu().numpy()
    cnt = step.selector.counts.cpu().numpy()
    scores = step.selector.page_scores.cpu()

    # the GPU selection is the exact top-k of the GPU's own key-mean scores (draft rows)
    n_pages = (ctx + 15) // 16
    logical, c = topk_pages_per_head(scores[: B * H], np.repeat(n_pages, H), step.budget, 1)
    logical = logical.numpy().reshape(B, H, -1)
    for b in np.flatnonzero(dr):
        for g in range(H):
            k = int(c[b * H + g])
            assert cnt[b, g] == k
            assert sel[b, g, :k].tolist() == table[b][logical[b, g, :k]].tolist()

    # the oracle step on the same weights, caches and inputs, with the GPU's selection
    w_cpu = step.w.to("cpu")
    ref = odecode.decode_step(w_cpu, caches0, step.shape, ctx, ql, dr, table, step.tokens.cpu(),
                              budget=step.budget, refresh_layer=2, recent_pages=1, selected=init_sel,
                              counts=init_cnt, selection_override=(sel, cnt))
    for layer in range(step.shape.n_layer):
        qg, qr = cap[f"q{layer}"].float().cpu(), ref[f"q{layer}"].float()
        assert (qg - qr).abs().max() <= 0.05 * qr.abs().max(), f"layer {layer} q"
    # The page scores are the key-mean epilogue of the GPU's own refresh-layer q and cache: max over
    # the group's heads of q . mean(k) per page, in fp32 on the CPU from the same inputs.
    G = step.shape.n_head // H
    q2 = cap["q2"].float().cpu()
    kc = step.caches[2].float().cpu()
    qo = np.concatenate([[0], np.cumsum(ql)])
    for b in np.flatnonzero(dr):
        for g in range(H):
            n = int(n_pages[b])
            want = torch.empty(n)
            for pg in range(n):
                kmean = kc[int(table[b][pg]), 0, : min(16, int(ctx[b]) - 16 * pg), g].mean(0)
                want[pg] = (q2[int(qo[b]), g * G : (g + 1) * G] @ kmean).max()
            assert torch.allclose(scores[b * H + g, :n], want, rtol=1e-3, atol=1e-3)
    # Against the oracle's whole step: its q differs from the GPU's by the roundings of two layers
    # (held to 5% of the largest |q| above), and so do the scores.
    ps_ref = ref["page_scores"]
    for b in np.flatnonzero(dr):
        for g in range(H):
            s = b * H + g
            n = int(n_pages[b])
            assert (scores[s, :n] - ps_ref[s, :n]).abs().max() <= 0.05 * ps_ref[s, :n].abs().max()
    lg, lr = step.logits.float().cpu(), ref["logits"].float()
    assert torch.isfinite(lg).all()
    assert (lg - lr).abs().max() <= 0.05 * lr.abs().max()
    assert (lg - lr).abs().mean() <= 0.01 * lr.abs().mean()
    top2 = torch.topk(lr, 2, dim=-1).values
    clear = (top2[:, 0] - top2[:, 1]) > 0.05 * lr.abs().max()
    assert torch.equal(ids.cpu()[clear], ref["ids"][clear])
    assert torch.equal(ids.cpu(), odecode.argmax_rows(step.logits.cpu()))
    # the appended K/V rows: the GPU cache holds the oracle's within bf16 noise, elsewhere unchanged
    cg = step.caches.cpu().float()
    cr = caches0.float()
    assert (cg - cr).abs().max() <= 0.05 * cr.abs().max()
    changed = (step.caches.cpu() != caches0.cpu()).any(dim=(2, 3, 4, 5))
    assert int(changed.sum()) <= step.shape.n_layer * int(((ctx - 1) // 16 - (ctx - ql) // 16 + 1).sum())


@pytest.mark.parametrize("shape", SHAPES)
def test_decode_step_graph_replays_match_eager(gpu, shape):
    """The whole step recorded in one HIP graph: every replay equals the eager step from the
    same state (the draft selection carried from step to step), with eager work between."""
    say("decode step graph", shape)
    step, *_ = _small_step(gpu, budget=6, seed=3, shape=shape)
    state = [step.selector.selected, step.selector.counts, step.mixed_indices, step.mixed_indptr]
    saved = [t.clone() for t in state]

    def restore():
        for t, s in zip(state, saved):
            t.copy_(s)

    eager = []
    for _ in range(3):
        ids = step.forward().clone()
        eager.append((ids, step.logits.clone(), step.selector.selected.clone()))
    restore()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step.forward()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    restore()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gids = step.forward()
    glogits = step.logits
    restore()
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        e_ids, e_logits, e_sel = eager[i]
        assert torch.equal(gids, e_ids), f"replay {i} ids"
        assert torch.equal(glogits, e_logits), f"replay {i} logits"
        assert torch.equal(step.selector.selected, e_sel), f"replay {i} selection"
        _ = torch.randn(1000, device=gpu).sum().item()   # eager work between replays
