"""The drop-in boundary driven the way the reference drives it: the attention ops registered
with torch.library around the HIP wrappers (mylib::unified_decode, sparse_draft_runner.py:
599-612; the refresh layer's dump op, base.py:452-489) and the paged append
(mylib::update_kv_padded), called from one function compiled with
torch.compile(fullgraph=True) and then captured in a HIP graph (base.py:1692-1719,
sparse_draft_runner.py:918-987). Eager, compiled and every graph replay must agree bit for
bit, and the outputs must match the oracle."""

import numpy as np
import pytest
import torch

import aspire_amd.attention.kv_ops  # noqa: F401  (registers mylib::update_kv_padded)
from aspire_amd.attention.holistic_wrapper import (HolisticAttentionWrapper, build_holistic_dump_jit_args,
                                                   define_dump_op, define_unified_decode_op)
from aspire_amd.workloads import PAGE, build_step
from helpers import attn_close, say
from oracle.attention import DumpSpec, paged_attention

pytestmark = pytest.mark.gpu


def test_compiled_and_captured_layer_matches_eager_and_oracle(gpu):
    say("torch.compile(fullgraph) + graph capture of the attention ops")
    H, HKV, stride = 16, 8, 1024
    kw = dict(hq=H, hkv=HKV, ctx_len=[900, 700, 1000, 333], q_len=[1, 1, 5, 3], draft_budget=12, seed=5,
              device=gpu)
    mixed = build_step(is_draft=[1, 1, 0, 0], **kw)     # draft rows over 12 selected pages
    full = build_step(is_draft=[0, 0, 0, 0], **kw)      # same seed and lengths: same cache, q and new K/V
    assert torch.equal(mixed.cache, full.cache) and torch.equal(mixed.q, full.q)
    B, T = mixed.batch, mixed.total_tokens

    w_mixed = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD", use_cuda_graph=True)
    w_mixed.plan(mixed.qo_indptr, mixed.kv_indptr, mixed.kv_indices, mixed.last_page_len, H, HKV, 128, PAGE,
                 causal=True)
    args = build_holistic_dump_jit_args(torch.bfloat16, 128, dump_kind="first_last_compact",
                                        dump_buffer_dtype=torch.float16)
    w_full = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD", use_cuda_graph=True, jit_args=args)
    w_full.plan(full.qo_indptr, full.kv_indptr, full.kv_indices, full.last_page_len, H, HKV, 128, PAGE,
                causal=True)
    unified = define_unified_decode_op(w_mixed, "mylib::unified_decode")
    dump_op = define_dump_op(w_full, "mylib::unified_full_decode_first_last_0", H, stride)

    # the full lists address every row's pages, a superset of the draft lists: append through them
    app = (full.qo_indptr, full.kv_indices, full.kv_indptr, full.last_page_len)

    def layer(q, k_new, v_new, kv_cache, out, out_full, dump):
        torch.ops.mylib.update_kv_padded(k_new, v_new, app[0], kv_cache, app[1], app[2], app[3], PAGE)
        unified(q, kv_cache, out)
        return dump_op(q, kv_cache, dump, out_full)

    def fresh():
        return (mixed.cache.clone(), torch.zeros_like(mixed.q), torch.zeros_like(mixed.q),
                torch.full((B * H * 2 * stride,), float("-inf"), dtype=torch.float16, device=gpu))

    cache_e, out_e, full_e, dump_e = fresh()
    lse_e = layer(mixed.q, mixed.k_new, mixed.v_new, cache_e, out_e, full_e, dump_e).clone()
    torch.cuda.synchronize()

    compiled = torch.compile(layer, fullgraph=True)
    cache_c, out_c, full_c, dump_c = fresh()
    lse_c = compiled(mixed.q, mixed.k_new, mixed.v_new, cache_c, out_c, full_c, dump_c)
    torch.cuda.synchronize()
    for name, a, b in (("cache", cache_c, cache_e), ("out", out_c, out_e), ("out_full", full_c, full_e),
                       ("dump", dump_c, dump_e), ("lse", lse_c, lse_e)):
        assert torch.equal(a, b), f"compiled {name} differs from eager"

    # capture the compiled layer (warm-up on a side stream first, as torch.cuda.graph expects)
    cache_g, out_g, full_g, dump_g = fresh()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        compiled(mixed.q, mixed.k_new, mixed.v_new, cache_g, out_g, full_g, dump_g)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        lse_g = compiled(mixed.q, mixed.k_new, mixed.v_new, cache_g, out_g, full_g, dump_g)
    for rep in range(3):
        cache_g.copy_(mixed.cache)
        out_g.zero_()
        full_g.zero_()
        dump_g.fill_(float("-inf"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in (("cache", cache_g, cache_e), ("out", out_g, out_e), ("out_full", full_g, full_e),
                           ("dump", dump_g, dump_e), ("lse", lse_g, lse_e)):
            assert torch.equal(a, b), f"replay {rep}: {name} differs from eager"
        _ = torch.randn(1000, device=gpu).sum().item()     # eager work between replays

    # and the eager results against the oracle
    cache = cache_e.cpu()
    ref, _ = paged_attention(mixed.q.cpu(), cache, mixed.qo_indptr_host, mixed.kv_indptr_host,
                             mixed.kv_indices.cpu(), mixed.kv_len_host, num_kv_heads=HKV)
    attn_close(out_e[:T], ref[:T])
    ref_dump = torch.full((B * H * 2 * stride,), float("-inf"), dtype=torch.float16)
    ref_full, ref_lse = paged_attention(full.q.cpu(), cache, full.qo_indptr_host, full.kv_indptr_host,
                                        full.kv_indices.cpu(), full.kv_len_host, num_kv_heads=HKV,
                                        dump=DumpSpec(buffer=ref_dump, kind="first_last", num_heads=H,
                                                      kv_stride=stride))
    attn_close(full_e[:T], ref_full[:T])
    assert (lse_e[:T].cpu() - ref_lse[:T]).abs().max() < 2e-3
    got, want = dump_e.cpu().float(), ref_dump.float()
    written = torch.isfinite(want)
    assert torch.equal(torch.isfinite(got), written)
    assert torch.allclose(got[written], want[written], rtol=2e-3, atol=2e-3)
    # the appended tokens are in the cache (the draft rows' current pages are in both lists)
    assert not torch.equal(cache_e, mixed.cache)
    np.testing.assert_array_equal(np.asarray(full.kv_len_host[:B]), np.asarray(mixed.ctx_len))
