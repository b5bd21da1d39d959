"""Mixed draft/verify attention on the GPU against the CPU oracle."""

import math

import numpy as np
import pytest
import torch

import aspire_amd.attention.kv_ops  # noqa: F401
from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper, build_holistic_dump_jit_args
from aspire_amd.workloads import PAGE, build_step, config0, config1
from helpers import attn_close, say
from oracle.attention import DumpSpec, paged_attention

pytestmark = pytest.mark.gpu


def make_wrapper(gpu, **kw):
    return HolisticAttentionWrapper(torch.empty(1, dtype=torch.uint8, device=gpu), "NHD", **kw)


def plan(w, step, causal=True):
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, step.hq, step.hkv, 128, PAGE,
           causal=causal)


def oracle(step, cache, causal=True, **kw):
    return paged_attention(step.q.cpu(), cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                           step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=step.hkv, causal=causal, **kw)


def check_rows(step, out, lse, ref_out, ref_lse):
    T = step.total_tokens
    attn_close(out[:T], ref_out[:T])
    l, rl = lse[:T].cpu(), ref_lse[:T]
    fin = torch.isfinite(rl)
    assert torch.equal(torch.isfinite(l), fin)
    assert (l[fin] - rl[fin]).abs().max().item() < 2e-3


def test_config0_step_append_then_attention(gpu):
    say("config0 append+attention")
    step = config0(device=gpu)
    cache = step.cache.clone()
    torch.ops.mylib.update_kv_padded(step.k_new, step.v_new, step.qo_indptr, cache, step.kv_indices,
                                     step.kv_indptr, step.last_page_len, PAGE)
    w = make_wrapper(gpu)
    plan(w, step)
    out, lse = w.run(step.q, cache, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = oracle(step, cache)
    check_rows(step, out, lse, ref_out, ref_lse)


CASES = [
    # name, hq, hkv, ctx, q_len, draft
    ("gqa4_mixed_ragged", 32, 8, [37, 16, 1, 500, 4096 + 5, 33], [1, 2, 1, 4, 3, 1], [1, 0, 1, 0, 0, 1]),
    ("gqa4_tile2_tile3", 32, 8, [700, 1025, 64, 3000], [5, 8, 9, 12], [0, 0, 0, 0]),
    ("gqa2_qwen17b", 16, 8, [4096, 4096, 1000, 77], [1, 5, 7, 16], [1, 0, 0, 0]),
    ("mha_gqa1", 8, 8, [129, 250], [3, 16], [0, 0]),
    ("gqa8", 64, 8, [300, 999], [2, 6], [0, 0]),
    # 3-tile items whose tiles run on two waves of a head: GQA 2 (tile 2 holds tokens 16..23),
    # 4 kv heads (a slot of one workgroup), and 2 kv heads (not head-aligned: every lane of a
    # split item loads its own pages)
    ("gqa2_tile3_split", 16, 8, [2000, 333, 4097], [24, 17, 20], [0, 0, 0]),
    ("gqa4_hkv4_tile3", 16, 4, [3000, 1000, 40], [9, 12, 11], [0, 0, 0]),
    ("gqa8_hkv2_direct_tile3", 16, 2, [1500, 700], [5, 6], [0, 0]),
]


@pytest.mark.parametrize("name,hq,hkv,ctx,qlen,draft", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("waves_per_cu", [8, 1])
def test_edge_shapes_match_oracle(gpu, name, hq, hkv, ctx, qlen, draft, waves_per_cu):
    say("attention", name, "waves_per_cu", waves_per_cu)
    step = build_step(hq=hq, hkv=hkv, ctx_len=ctx, q_len=qlen, is_draft=draft, draft_budget=9, seed=3,
                      device=gpu, bucket_tokens=sum(qlen) + 2)
    T = int(step.qo_indptr_host[-1])
    q = torch.randn(T, hq, 128, device=gpu).bfloat16()
    q[: step.total_tokens] = step.q
    step.q = q
    w = make_wrapper(gpu, waves_per_cu=waves_per_cu)
    plan(w, step)
    out, lse = w.run(step.q, step.cache, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = oracle(step, step.cache)
    check_rows(step, out, lse, ref_out, ref_lse)
    # bucket-padding tokens (the trailing row with no pages) get zeros and lse = -inf
    assert (out[step.total_tokens:].float() == 0).all()
    assert torch.isinf(lse[step.total_tokens:]).all()


def test_non_causal_and_explicit_scale(gpu):
    say("non-causal")
    step = build_step(hq=32, hkv=8, ctx_len=[300, 64], q_len=[4, 2], is_draft=[0, 0], draft_budget=0, seed=5,
                      device=gpu)
    w = make_wrapper(gpu)
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 32, 8, 128, PAGE, causal=False,
           sm_scale=0.05)
    out, lse = w.run(step.q, step.cache, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = oracle(step, step.cache, causal=False, sm_scale=0.05)
    check_rows(step, out, lse, ref_out, ref_lse)


def test_plan_host_matches_plan_and_split_is_invisible(gpu):
    say("plan_host + split")
    step = build_step(hq=32, hkv=8, ctx_len=[20000, 9000, 2048], q_len=[1, 4, 1], is_draft=[0, 0, 1],
                      draft_budget=32, seed=8, device=gpu)
    w1 = make_wrapper(gpu, waves_per_cu=8)
    plan(w1, step)
    w1.plan_host(step.qo_indptr_host, step.kv_indptr_host, step.kv_len_host, step.kv_indices, 32, 8, 128, PAGE,
                 causal=True)
    assert w1.plan_info.num_merge > 0
    a = w1.run(step.q, step.cache)
    w2 = make_wrapper(gpu, waves_per_cu=1)
    plan(w2, step)
    b = w2.run(step.q, step.cache)
    torch.cuda.synchronize()
    ref_out, _ = oracle(step, step.cache)
    attn_close(a, ref_out)
    attn_close(b, ref_out)


def test_plan_host_requires_plan(gpu):
    w = make_wrapper(gpu)
    step = config0(device=gpu)
    with pytest.raises(RuntimeError, match="prior plan"):
        w.plan_host(step.qo_indptr_host, step.kv_indptr_host, step.kv_len_host, step.kv_indices, 16, 8, 128, PAGE)


def test_page_pool_permutation_is_bitwise_invisible(gpu):
    say("pool permutation")
    step = config0(device=gpu)
    w = make_wrapper(gpu)
    plan(w, step)
    out1 = w.run(step.q, step.cache).clone()
    P = step.cache.shape[0]
    perm = torch.randperm(P, generator=torch.Generator().manual_seed(1)).to(gpu)
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(P, device=gpu)
    cache2 = step.cache[perm]
    idx2 = inv[step.kv_indices.long()].to(torch.int32)
    w.plan(step.qo_indptr, step.kv_indptr, idx2, step.last_page_len, 16, 8, 128, PAGE, causal=True)
    out2 = w.run(step.q, cache2)
    torch.cuda.synchronize()
    assert torch.equal(out1, out2)


def test_per_head_page_lists(gpu):
    say("per-head lists")
    B, hq, hkv = 3, 32, 8
    step = build_step(hq=hq, hkv=hkv, ctx_len=[1600, 800, 3000], q_len=[1, 1, 1], is_draft=[0, 0, 0],
                      draft_budget=0, seed=11, device=gpu)
    rng = np.random.default_rng(0)
    table = step.block_table.cpu().numpy()
    kvp, lists, kvl = [0], [], []
    for b in range(B):
        n = (int(step.ctx_len[b]) + 15) // 16
        for g in range(hkv):
            k = int(rng.integers(1, n + 1))
            sel = np.sort(np.concatenate([rng.choice(n - 1, size=k - 1, replace=False), [n - 1]])) if k > 1 else np.array([n - 1])
            lists.append(table[b, sel])
            kvp.append(kvp[-1] + k)
            kvl.append((k - 1) * 16 + (int(step.ctx_len[b]) - 1) % 16 + 1)
    idx = torch.from_numpy(np.concatenate(lists).astype(np.int32)).to(gpu)
    qo = torch.tensor([0, 1, 2, 3], dtype=torch.int32)
    w = make_wrapper(gpu)
    plan(w, step)
    w.plan_host(qo, torch.tensor(kvp, dtype=torch.int32), torch.tensor(kvl, dtype=torch.int32), idx, hq, hkv, 128,
                PAGE, causal=True, per_head_lists=True)
    out, lse = w.run(step.q, step.cache, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = paged_attention(step.q.cpu(), step.cache.cpu(), qo, kvp, idx.cpu(), kvl, num_kv_heads=hkv,
                                       per_head_lists=True)
    attn_close(out, ref_out)
    assert (lse.cpu() - ref_lse).abs().max() < 2e-3


@pytest.mark.parametrize("wpc", [None, 8])
def test_segment_plan_shared_and_per_head_rows(gpu, wpc):
    """plan_segments: verify rows share one list across heads (staged path), draft rows
    read one list per head (direct path) in the same head-aligned launch."""
    say("segment plan", wpc)
    hq, hkv = 32, 8
    ctx = np.array([3000, 1000, 2500, 700, 4000, 333, 1600])
    ql = np.array([1, 4, 1, 9, 1, 7, 2])
    draft = ql == 1
    step = build_step(hq=hq, hkv=hkv, ctx_len=ctx, q_len=ql, is_draft=[0] * len(ctx), draft_budget=0, seed=21,
                      device=gpu)
    table = step.block_table.cpu().numpy()
    rng = np.random.default_rng(7)
    n_pages = (ctx + 15) // 16
    last = (ctx - 1) % 16 + 1
    idx, start, pages, kvl = [], [], [], []
    pos = 0
    for b in range(len(ctx)):
        n = int(n_pages[b])
        if draft[b]:
            k = min(24, n)
            for g in range(hkv):
                sel = np.sort(np.concatenate([rng.choice(n - 1, size=k - 1, replace=False), [n - 1]]))
                idx.append(table[b, sel])
                start.append(pos)
                pos += k
                pages.append(k)
                kvl.append((k - 1) * 16 + last[b])
        else:
            idx.append(table[b, :n])
            start += [pos] * hkv
            pages += [n] * hkv
            kvl += [int(ctx[b])] * hkv
            pos += n
    flat = np.concatenate(idx).astype(np.int32)
    w = make_wrapper(gpu, waves_per_cu=wpc)
    plan(w, step)
    t32 = lambda a: torch.tensor(np.asarray(a), dtype=torch.int32)
    w.plan_segments(step.qo_indptr_host[: len(ctx) + 1], t32(start), t32(pages), t32(kvl),
                    torch.from_numpy(flat).to(gpu), hq, hkv, 128, PAGE, causal=True)
    out, lse = w.run(step.q, step.cache, return_lse=True)
    torch.cuda.synchronize()
    # the oracle takes per-head lists laid end to end
    kvp_o = np.concatenate([[0], np.cumsum(pages)])
    idx_o = np.concatenate([flat[s0 : s0 + n] for s0, n in zip(start, pages)])
    ref_out, ref_lse = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host[: len(ctx) + 1], kvp_o,
                                       torch.from_numpy(idx_o), kvl, num_kv_heads=hkv, per_head_lists=True)
    T = int(ql.sum())
    attn_close(out[:T], ref_out[:T])
    assert (lse[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3


@pytest.mark.parametrize("kind,dtype,shape", [
    ("first_last_compact", torch.float16, "small"), ("last_token", torch.float16, "small"),
    ("first_last_compact", torch.float32, "long"), ("last_token", torch.float16, "long"),
    ("last_token", torch.float16, "odd_stride")])
def test_logits_dump(gpu, kind, dtype, shape):
    """Dump entries against the oracle's, fp16 and fp32: 8- or 16-byte stores of a lane's 4 keys
    when the row stride is a multiple of 4 (one store per key otherwise, and on a partial last
    group). The long case (GQA 4, contexts of 4,099 / 535 / 9,000 tokens, a single-query row
    beside 5- and 9-token rows of 2 and 3 tiles) splits rows into many pieces."""
    say("dump", kind, dtype, shape)
    if shape == "long":
        step = build_step(hq=32, hkv=8, ctx_len=[4099, 535, 9000], q_len=[1, 5, 9], is_draft=[0, 0, 0],
                          draft_budget=0, seed=21, device=gpu)
        H, stride = 32, 9216
    else:
        step = build_step(hq=16, hkv=8, ctx_len=[500, 77, 1000], q_len=[5, 1, 3], is_draft=[0, 0, 0],
                          draft_budget=0, seed=12, device=gpu)
        H, stride = 16, 1024 if shape == "small" else 1023
    B = step.batch
    slots = 2 if kind == "first_last_compact" else 1
    args = build_holistic_dump_jit_args(torch.bfloat16, 128, dump_kind=kind, dump_buffer_dtype=dtype)
    w = make_wrapper(gpu, jit_args=args)
    plan(w, step)
    dump = torch.full((B * H * slots * stride,), float("-inf"), dtype=dtype, device=gpu)
    out, lse = w.run(step.q, step.cache, dump, H, stride, return_lse=True)
    torch.cuda.synchronize()
    ref_dump = torch.full((B * H * slots * stride,), float("-inf"), dtype=dtype)
    ref_out, ref_lse = oracle(step, step.cache, dump=DumpSpec(buffer=ref_dump, kind=kind.replace("_compact", ""),
                                                                num_heads=H, kv_stride=stride))
    check_rows(step, out, lse, ref_out, ref_lse)
    got = dump.cpu().float()
    ref = ref_dump.float()
    written = torch.isfinite(ref)
    assert torch.equal(torch.isfinite(got), written), "dump wrote outside the reference's entries"
    # raw q.k in fp32 then fp16: equal up to one fp16 rounding step
    assert torch.allclose(got[written], ref[written], rtol=2e-3, atol=2e-3)


def test_dump_mode_flags(gpu):
    step = build_step(hq=16, hkv=8, ctx_len=[100, 100], q_len=[2, 2], is_draft=[0, 0], draft_budget=0, seed=2,
                      device=gpu)
    args = build_holistic_dump_jit_args(torch.bfloat16, 128, dump_kind="first_last_compact", use_mode_flags=True,
                                        dump_buffer_dtype=torch.float16)
    w = make_wrapper(gpu, jit_args=args)
    plan(w, step)
    dump = torch.full((2 * 16 * 2 * 128,), float("-inf"), dtype=torch.float16, device=gpu)
    flags = torch.tensor([0, 1], dtype=torch.int32, device=gpu)
    w.run(step.q, step.cache, dump, flags, 16, 128)
    torch.cuda.synchronize()
    v = dump.view(2, 16, 2, 128)
    assert torch.isinf(v[0]).all() and torch.isfinite(v[1, :, :, :100]).all()


def test_keymean_page_scores(gpu):
    say("key-mean page scores")
    step = build_step(hq=32, hkv=8, ctx_len=[1000, 2048, 37], q_len=[1, 1, 1], is_draft=[0, 0, 0], draft_budget=0,
                      seed=13, device=gpu)
    w = make_wrapper(gpu)
    plan(w, step)
    scores = torch.full((3 * 8, 128), float("nan"), device=gpu)
    w.run(step.q, step.cache, page_scores=scores)
    torch.cuda.synchronize()
    ref = torch.full((3 * 8, 128), float("nan"))
    oracle(step, step.cache, page_scores=ref)
    fin = ~torch.isnan(ref)
    assert torch.equal(~torch.isnan(scores.cpu()), fin)
    assert torch.allclose(scores.cpu()[fin], ref[fin], rtol=1e-4, atol=1e-4)


def test_graph_capture_replays_new_plans(gpu):
    say("graph capture")
    steps = [build_step(hq=32, hkv=8, ctx_len=c, q_len=q, is_draft=[0] * len(c), draft_budget=0, seed=s,
                        device=gpu, pool_pages=4096, bucket_tokens=16)
             for s, (c, q) in enumerate([([3000, 500, 70], [4, 1, 2]), ([200, 5000, 1000], [1, 4, 4]),
                                         ([16, 8000, 33], [2, 2, 1])])]
    w = make_wrapper(gpu, use_cuda_graph=True)
    # static buffers the graph reads
    q_buf = torch.zeros(16, 32, 128, dtype=torch.bfloat16, device=gpu)
    out_buf = torch.zeros_like(q_buf)
    idx_buf = torch.zeros(4096, dtype=torch.int32, device=gpu)
    cache = steps[0].cache

    def stage(st):
        q_buf.zero_()
        q_buf[: st.total_tokens] = st.q
        idx_buf[: st.kv_indices.numel()] = st.kv_indices
        cache.copy_(st.cache)
        w.plan(st.qo_indptr, st.kv_indptr, idx_buf, st.last_page_len, 32, 8, 128, PAGE, causal=True)

    stage(steps[0])
    w.run(q_buf, cache, out=out_buf)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w.run(q_buf, cache, out=out_buf)
    for rep in range(2):
        for st in steps:
            stage(st)
            g.replay()
            torch.cuda.synchronize()
            got = out_buf[: st.total_tokens].clone()
            eager = w.run(q_buf, cache)[: st.total_tokens]
            torch.cuda.synchronize()
            assert torch.equal(got, eager)
            ref_out, _ = paged_attention(st.q.cpu(), cache.cpu(), st.qo_indptr_host, st.kv_indptr_host,
                                         st.kv_indices.cpu(), st.kv_len_host, num_kv_heads=8)
            attn_close(got, ref_out[: st.total_tokens])


def test_config1_full_size_sampled_rows(gpu):
    say("config1 full size")
    step = config1(device=gpu)
    cache = step.cache
    torch.ops.mylib.update_kv_padded(step.k_new, step.v_new, step.qo_indptr, cache, step.kv_indices,
                                     step.kv_indptr, step.last_page_len, PAGE)
    w = make_wrapper(gpu)
    plan(w, step)
    out, lse = w.run(step.q, cache, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all() and torch.isfinite(lse).all()
    # oracle on a sample of rows (two draft, two verify) through a reduced plan
    rows = [0, 15, 16, 31]
    qo = step.qo_indptr_host.numpy()
    kvp = step.kv_indptr_host.numpy()
    kvl = step.kv_len_host.numpy()
    idx = step.kv_indices.cpu()
    sub_qo, sub_kvp, sub_kvl, sub_idx, toks = [0], [0], [], [], []
    for b in rows:
        toks += list(range(qo[b], qo[b + 1]))
        sub_qo.append(sub_qo[-1] + qo[b + 1] - qo[b])
        sub_idx.append(idx[kvp[b] : kvp[b + 1]])
        sub_kvp.append(sub_kvp[-1] + kvp[b + 1] - kvp[b])
        sub_kvl.append(kvl[b])
    used = torch.cat(sub_idx).long()
    uniq, inv = torch.unique(used, return_inverse=True)
    small_cache = cache[uniq.to(gpu)].cpu()
    ref_out, ref_lse = paged_attention(step.q[toks].cpu(), small_cache, sub_qo, sub_kvp, inv.to(torch.int32),
                                       sub_kvl, num_kv_heads=8)
    attn_close(out[toks], ref_out)
    assert (lse[toks].cpu() - ref_lse).abs().max() < 2e-3


def test_small_layout_merge_reads_stay_in_plan(gpu):
    """A layout for few waves with a small int workspace holds fewer merge items (291) than
    the merge launch has waves per item slot (4,096 waves / 12 tasks per item): every wave's
    first-item read must stay inside the plan's merge region, and the split rows merge
    correctly. The device buffer is exactly the layout's size."""
    import ctypes

    from aspire_amd import _lib

    say("small layout merge")
    lay = _lib.PlanLayout()
    _lib.check(_lib.lib().aspire_plan_layout_init(8, 4, 40 << 10, 64 << 20, 128, ctypes.byref(lay)), "layout")
    assert lay.max_merge * 12 < 4096, lay.max_merge
    step = build_step(hq=32, hkv=8, ctx_len=[20000, 9000, 2048, 15000], q_len=[1, 4, 1, 9], is_draft=[0, 0, 1, 0],
                      draft_budget=32, seed=21, device=gpu)
    qo = np.ascontiguousarray(step.qo_indptr_host.numpy(), dtype=np.int32)
    kvp = np.ascontiguousarray(step.kv_indptr_host.numpy(), dtype=np.int32)
    kvl = np.ascontiguousarray(step.kv_len_host.numpy()[: step.batch], dtype=np.int32)
    buf = np.zeros(lay.int_ws_bytes // 4, dtype=np.int32)
    info = _lib.PlanInfo()
    _lib.check(_lib.lib().aspire_plan_build(
        ctypes.byref(lay), qo.ctypes.data_as(ctypes.c_void_p), kvp.ctypes.data_as(ctypes.c_void_p),
        kvl.ctypes.data_as(ctypes.c_void_p), step.batch, 0, step.hq, step.hkv, PAGE, 1,
        buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes, ctypes.byref(info)), "plan")
    assert info.num_merge > 0
    plan_dev = torch.from_numpy(buf).to(gpu)
    float_ws = torch.empty(lay.float_ws_bytes // 4, dtype=torch.float32, device=gpu)
    T = step.total_tokens
    out = torch.full_like(step.q, float("nan"))
    k_cache, v_cache = step.cache[:, 0], step.cache[:, 1]
    a = _lib.AttentionArgs()
    a.q, a.q_stride_t, a.q_stride_h = step.q.data_ptr(), step.q.stride(0), step.q.stride(1)
    a.kv_cache, a.cache_stride_p = k_cache.data_ptr(), k_cache.stride(0)
    a.cache_stride_kv = (v_cache.data_ptr() - k_cache.data_ptr()) // 2
    a.cache_stride_t, a.cache_stride_h = k_cache.stride(1), k_cache.stride(2)
    a.kv_indices = step.kv_indices.data_ptr()
    a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.lse = None
    a.plan_dev, a.float_ws = plan_dev.data_ptr(), float_ws.data_ptr()
    a.num_qo_heads, a.num_kv_heads, a.head_dim, a.page_size = step.hq, step.hkv, 128, PAGE
    a.sm_scale, a.causal, a.class_mask, a.launch_merge = 1.0 / 128 ** 0.5, 1, 7, 1
    _lib.check(_lib.lib().aspire_attention_run(ctypes.byref(lay), ctypes.byref(a), _lib.stream_of(step.q)), "run")
    torch.cuda.synchronize()
    ref, _ = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                             step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=step.hkv)
    attn_close(out[:T], ref[:T])


@pytest.mark.parametrize("ctx,q_len,draft", [
    ([20000, 9000, 2048, 15000], [1, 4, 1, 9], [0, 0, 1, 0]),   # a short plan: few pages per wave
    ([8192] * 24, [1, 4, 9] * 8, [1, 0, 0] * 8),               # longer: ~90 page-heads per wave
])
def test_partial_store_kinds_are_bitwise_identical(gpu, monkeypatch, ctx, q_len, draft):
    """run() stores the split-KV partials non-temporally for plans of at most
    SHORT_PLAN_PAGES_PER_WAVE page-heads per wave and with plain stores otherwise; the two kernel
    instances write the same values, so forcing either choice gives bit-equal outputs and LSEs."""
    from aspire_amd.attention import holistic_wrapper as hw

    say("partial store kinds", len(ctx))
    step = build_step(hq=32, hkv=8, ctx_len=ctx, q_len=q_len, is_draft=draft, draft_budget=64, seed=23, device=gpu)
    w = make_wrapper(gpu)
    plan(w, step)
    assert w.plan_info.num_merge > 0
    short = w.plan_info.total_pages <= hw.SHORT_PLAN_PAGES_PER_WAVE * w._layout.num_waves
    assert short == (len(ctx) == 4)
    res = {}
    for limit in (0, 1 << 30):  # plain, then non-temporal partial stores
        monkeypatch.setattr(hw, "SHORT_PLAN_PAGES_PER_WAVE", limit)
        out, lse = w.run(step.q, step.cache, return_lse=True)
        torch.cuda.synchronize()
        res[limit] = (out.clone(), lse.clone())
    (o0, l0), (o1, l1) = res[0], res[1 << 30]
    T = step.total_tokens
    assert torch.equal(o0[:T].view(torch.int16), o1[:T].view(torch.int16))
    assert torch.equal(l0[:T], l1[:T])
    ref_out, ref_lse = oracle(step, step.cache)
    check_rows(step, o1, l1, ref_out, ref_lse)
