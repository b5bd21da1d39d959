"""Chunked prefill through the paged path (BatchPrefillWithPagedKVCacheWrapper drop-in) against the oracle."""

import pytest
import torch

from aspire_amd import _lib
from aspire_amd.attention.holistic_wrapper import build_holistic_dump_jit_args
from aspire_amd.attention.prefill import BatchPrefillWithPagedKVCacheWrapper
from aspire_amd.workloads import PAGE, build_step
from helpers import attn_close, say
from oracle.attention import paged_attention

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kernel", ["prefill", "decode"])
@pytest.mark.parametrize("causal", [True, False])
def test_chunked_prefill_matches_oracle(gpu, causal, kernel):
    """Prompt chunks over cached prefixes (as encode_slots plans them): 300 new tokens over 700 cached,
    a 1000-token first chunk, 64 over 4000, and a decode row, Qwen3-8B heads (GQA 4); through the
    dedicated prefill kernel and through the decode kernel's query tiles."""
    say("prefill", causal, kernel)
    step = build_step(hq=32, hkv=8, ctx_len=[1000, 1000, 4064, 5000], q_len=[300, 1000, 64, 1],
                      is_draft=[0, 0, 0, 0], draft_budget=0, seed=31, device=gpu)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=gpu), "NHD", kernel=kernel)
    w.plan(qo_indptr=step.qo_indptr, paged_kv_indptr=step.kv_indptr, paged_kv_indices=step.kv_indices,
           paged_kv_last_page_len=step.last_page_len, num_qo_heads=32, num_kv_heads=8, head_dim_qk=128,
           page_size=PAGE, q_data_type=torch.bfloat16, causal=causal)
    assert w.plan_info.split_rows == 3
    out, lse = w.run(step.q, step.cache, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                                       step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=8, causal=causal)
    T = step.total_tokens
    attn_close(out[:T], ref_out[:T])
    assert (lse[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3


def test_dump_refuses_split_rows(gpu):
    step = build_step(hq=16, hkv=8, ctx_len=[200], q_len=[100], is_draft=[0], draft_budget=0, seed=2, device=gpu)
    args = build_holistic_dump_jit_args(torch.bfloat16, 128, dump_kind="first_last_compact",
                                        dump_buffer_dtype=torch.float16)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=gpu), "NHD", jit_args=args)
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 16, 8, 128, PAGE, causal=True)
    dump = torch.zeros(16 * 2 * 256, dtype=torch.float16, device=gpu)
    with pytest.raises(ValueError, match="whole rows"):
        w.run(step.q, step.cache, dump, 16, 256)


@pytest.mark.parametrize("hq,hkv", [(32, 8), (16, 8), (8, 8), (64, 8), (64, 2)])
def test_prefill_kernel_head_groups_and_edges(gpu, hq, hkv):
    """GQA groups 4, 2, 1, 8 and 32 (query blocks of 32, 64, 128, 16 and 4 tokens), rows that end mid-block
    and mid-page, a row whose chunk starts at position 0, one with a single new token, and a tail page
    with one valid key; stale slots past each row's length hold NaN keys and +inf values."""
    say("prefill kernel edges", hq, hkv)
    step = build_step(hq=hq, hkv=hkv, ctx_len=[257, 3001, 130, 16 * 40 + 1, 77], q_len=[257, 333, 1, 129, 20],
                      is_draft=[0] * 5, draft_budget=0, seed=32, device=gpu)
    cache = step.cache.clone()
    table = step.block_table.cpu().numpy()
    for b, n in enumerate(step.ctx_len):
        last = (int(n) - 1) % PAGE + 1
        if last < PAGE:
            page = int(table[b, (int(n) - 1) // PAGE])
            cache[page, 0, last:] = float("nan")
            cache[page, 1, last:] = float("inf")
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=gpu), "NHD")
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, hq, hkv, 128, PAGE, causal=True)
    assert w._pf is not None
    out, lse = w.run(step.q, cache, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                                       step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=hkv, causal=True)
    T = step.total_tokens
    attn_close(out[:T], ref_out[:T])
    assert (lse[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3


def test_prefill_kernel_separate_kv_tensors_and_gqa16(gpu):
    """K and V in two tensors (the (k_cache, v_cache) form, so the K-to-V distance is an
    arbitrary allocation offset), and GQA 16 (8-token query blocks)."""
    say("prefill kernel separate k/v, GQA 16")
    step = build_step(hq=32, hkv=2, ctx_len=[700, 129, 40], q_len=[300, 129, 7], is_draft=[0] * 3, draft_budget=0,
                      seed=33, device=gpu)
    k_cache = step.cache[:, 0].contiguous()
    v_cache = step.cache[:, 1].contiguous()
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=gpu), "NHD")
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 32, 2, 128, PAGE, causal=True)
    assert w._pf is not None and w._pf["block_tokens"] * 16 == _lib.lib().aspire_prefill_block_tokens(1, 1)
    out, lse = w.run(step.q, (k_cache, v_cache), return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                                       step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=2, causal=True)
    T = step.total_tokens
    attn_close(out[:T], ref_out[:T])
    assert (lse[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_kernel_full_chunk_matches_decode_path(gpu, causal):
    """The reference's largest prompt chunk (8,192 tokens, Qwen3-8B heads) at full size: the
    dedicated kernel against the decode kernel's query tiles, which the tests above pin to the
    oracle on the same rule (the CPU oracle at this size would take minutes)."""
    say("prefill 8192 chunk vs decode path", causal)
    step = build_step(hq=32, hkv=8, ctx_len=[8192], q_len=[8192], is_draft=[0], draft_budget=0, seed=34, device=gpu)
    res = {}
    for kernel in ("prefill", "decode"):
        w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=gpu), "NHD", kernel=kernel)
        w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 32, 8, 128, PAGE, causal=causal)
        res[kernel] = w.run(step.q, step.cache, return_lse=True)
        torch.cuda.synchronize()
    (out_p, lse_p), (out_d, lse_d) = res["prefill"], res["decode"]
    attn_close(out_p, out_d)
    assert (lse_p - lse_d).abs().max().item() < 2e-3


def test_prefill_head_group_outside_the_kernel_takes_the_decode_path(gpu):
    """GQA 6 (24 query heads over 4 kv heads) does not divide the prefill kernel's 32 query
    rows per wave: plan() routes the rows to the mixed kernel's query tiles, same results."""
    say("prefill GQA 6")
    step = build_step(hq=24, hkv=4, ctx_len=[500, 90], q_len=[200, 90], is_draft=[0, 0], draft_budget=0, seed=35,
                      device=gpu)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=gpu), "NHD")
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 24, 4, 128, PAGE, causal=True)
    assert w._pf is None
    out, lse = w.run(step.q, step.cache, return_lse=True)
    torch.cuda.synchronize()
    ref_out, ref_lse = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                                       step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=4, causal=True)
    T = step.total_tokens
    attn_close(out[:T], ref_out[:T])
    assert (lse[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3


def _plan_arrays(table: torch.Tensor, q_lens, kv_lens):
    """Reference-layout plan arrays of rows over prefixes of ``table``'s rows (host tensors)."""
    npg = [(int(n) + PAGE - 1) // PAGE for n in kv_lens]
    qo = torch.tensor([0, *torch.cumsum(torch.tensor(q_lens), 0).tolist()], dtype=torch.int32)
    kvp = torch.tensor([0, *torch.cumsum(torch.tensor(npg), 0).tolist()], dtype=torch.int32)
    idx = torch.cat([table[b, :n].cpu() for b, n in enumerate(npg)]).to(torch.int32)
    lpl = torch.tensor([(int(n) - 1) % PAGE + 1 for n in kv_lens], dtype=torch.int32)
    return qo, kvp, idx, lpl


@pytest.mark.parametrize("use_cuda_graph", [True, False])
def test_prefill_wrapper_graph_replays_later_plans(gpu, use_cuda_graph):
    """The reference's decode/draft wrappers are this class with use_cuda_graph=True and fixed
    index buffers, captured once and replayed after every re-plan (sparse_draft_runner.py:261-268,
    297-303). A run captured after plan A must replay plan B (other query and key lengths, other
    page lists, written into the same buffers) exactly as the oracle computes B; a wrapper
    without use_cuda_graph that is captured anyway must do the same."""
    say("prefill wrapper graph replay", use_cuda_graph)
    step = build_step(hq=32, hkv=8, ctx_len=[2048, 1024, 704], q_len=[1, 1, 1], is_draft=[0, 0, 0],
                      draft_budget=0, seed=36, device=gpu)
    gen = torch.Generator(device=gpu).manual_seed(7)
    q_buf = torch.randn(16, 32, 128, generator=gen, device=gpu).to(torch.bfloat16)
    out_buf = torch.zeros_like(q_buf)
    cap = int(step.block_table.numel())
    qo_buf = torch.zeros(4, dtype=torch.int32, device=gpu)
    kvp_buf = torch.zeros(4, dtype=torch.int32, device=gpu)
    idx_buf = torch.zeros(cap, dtype=torch.int32, device=gpu)
    lpl_buf = torch.zeros(3, dtype=torch.int32, device=gpu)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=gpu), "NHD", use_cuda_graph=use_cuda_graph,
                                            qo_indptr_buf=qo_buf, paged_kv_indptr_buf=kvp_buf,
                                            paged_kv_indices_buf=idx_buf, paged_kv_last_page_len_buf=lpl_buf)
    cache_cpu = step.cache.cpu()

    def plan(q_lens, kv_lens):
        qo, kvp, idx, lpl = _plan_arrays(step.block_table, q_lens, kv_lens)
        qo_buf.copy_(qo)
        kvp_buf.copy_(kvp)
        idx_buf[: idx.numel()].copy_(idx)
        lpl_buf.copy_(lpl)
        w.plan(qo_buf, kvp_buf, idx_buf, lpl_buf, 32, 8, 128, PAGE, causal=True)
        ref_out, ref_lse = paged_attention(q_buf.cpu(), cache_cpu, qo, kvp, idx, list(kv_lens), num_kv_heads=8,
                                           causal=True)
        return int(qo[-1]), ref_out

    plan_a = ([1, 4, 2], [300, 1000, 64])
    plan_b = ([3, 1, 5], [2048, 90, 640])
    T, ref = plan(*plan_a)
    w.run(q_buf, step.cache, out=out_buf)  # eager warm-up before capture
    torch.cuda.synchronize()
    attn_close(out_buf[:T], ref[:T])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        w.run(q_buf, step.cache, out=out_buf)
    for q_lens, kv_lens in (plan_a, plan_b, plan_a):
        T, ref = plan(q_lens, kv_lens)
        out_buf.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        attn_close(out_buf[:T], ref[:T])
        # and the same plan eagerly (the prefill kernel when the wrapper is not in graph mode)
        out = w.run(q_buf, step.cache)
        torch.cuda.synchronize()
        attn_close(out[:T], ref[:T])
