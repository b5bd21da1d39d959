"""aspire_attention_run_static (the allocation-free attention entry point) against
aspire_attention_run, both called through the C ABI on the same plan.

The static variant keeps the split-KV partials in the library's static device
array instead of the caller's float workspace; with one plan and one input its
output and LSE must equal the workspace variant's bit for bit. Two calls in a
row, the second on a smaller batch, check that the array's leftover contents
from the first call never reach the second.
"""

import ctypes

import pytest
import torch

from aspire_amd import _lib
from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper
from aspire_amd.workloads import PAGE, build_step
from helpers import attn_close, bits, say
from oracle.attention import paged_attention

pytestmark = pytest.mark.gpu


def _args(w, step, out, lse, float_ws):
    k_cache, v_cache = step.cache[:, 0], step.cache[:, 1]
    a = _lib.AttentionArgs()
    a.q, a.q_stride_t, a.q_stride_h = step.q.data_ptr(), step.q.stride(0), step.q.stride(1)
    a.kv_cache = k_cache.data_ptr()
    a.cache_stride_p = k_cache.stride(0)
    a.cache_stride_kv = (v_cache.data_ptr() - k_cache.data_ptr()) // 2
    a.cache_stride_t, a.cache_stride_h = k_cache.stride(1), k_cache.stride(2)
    a.kv_indices = step.kv_indices.data_ptr()
    a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
    a.lse = lse.data_ptr()
    a.plan_dev = w._int_workspace.data_ptr()
    a.float_ws = float_ws
    a.num_qo_heads, a.num_kv_heads, a.head_dim, a.page_size = step.hq, step.hkv, 128, PAGE
    a.sm_scale, a.causal = 1.0 / 128 ** 0.5, 1
    a.class_mask, a.launch_merge = 7, 1
    return a


def _run(fn_name, w, a, like):
    rc = getattr(_lib.lib(), fn_name)(ctypes.byref(w._layout), ctypes.byref(a), _lib.stream_of(like))
    _lib.check(rc, fn_name)


def test_static_scratch_entry_matches_workspace_entry(gpu):
    # the wrapper's layout describes exactly the static array, so both entries run one plan
    w = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD", float_workspace_bytes=_lib.STATIC_SCRATCH_BYTES)
    assert w._layout.float_ws_bytes <= _lib.STATIC_SCRATCH_BYTES
    cases = [
        # larger first: GQA 4, drafts and verify rows up to the 3-tile class, long rows that split
        ("large", dict(hq=32, hkv=8, ctx_len=[8192, 6000, 8192, 5000, 7777, 4096, 8192, 3000],
                       q_len=[1, 4, 1, 9, 6, 1, 12, 2], is_draft=[1, 0, 1, 0, 0, 1, 0, 0], draft_budget=96, seed=11)),
        # then a smaller batch over the same static array
        ("small", dict(hq=32, hkv=8, ctx_len=[300, 2048, 77], q_len=[1, 5, 3], is_draft=[1, 0, 0],
                       draft_budget=8, seed=12)),
    ]
    for name, kw in cases:
        say(f"no-alloc entry: {name}")
        step = build_step(device=gpu, **kw)
        w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, step.hq, step.hkv, 128, PAGE,
               causal=True)
        if name == "large":
            assert w.plan_info.num_merge > 0 and w.plan_info.partial_rows > 0, "the case must split rows"
        T = step.total_tokens
        out_ws = torch.full_like(step.q, float("nan"))
        out_st = torch.full_like(step.q, float("nan"))
        lse_ws = torch.full((T, step.hq), float("nan"), device=gpu)
        lse_st = torch.full((T, step.hq), float("nan"), device=gpu)
        _run("aspire_attention_run", w, _args(w, step, out_ws, lse_ws, w._float_workspace.data_ptr()), step.q)
        _run("aspire_attention_run_static", w, _args(w, step, out_st, lse_st, None), step.q)
        torch.cuda.synchronize()
        assert (bits(out_st) == bits(out_ws)).all(), f"{name}: outputs differ"
        assert torch.equal(lse_st.cpu(), lse_ws.cpu()), f"{name}: lse differs"
        ref, _ = paged_attention(step.q.cpu(), step.cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                                 step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=step.hkv)
        attn_close(out_st[:T], ref[:T])


def test_static_scratch_entry_rejects_oversized_layouts(gpu):
    say("no-alloc entry: argument checks")
    step = build_step(hq=16, hkv=8, ctx_len=[64], q_len=[1], is_draft=[0], draft_budget=0, seed=1, device=gpu)
    out = torch.empty_like(step.q)
    lse = torch.empty(1, 16, device=gpu)
    big = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD")  # 384 MiB layout
    big.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 16, 8, 128, PAGE, causal=True)
    rc = _lib.lib().aspire_attention_run_static(ctypes.byref(big._layout), ctypes.byref(_args(big, step, out, lse, None)),
                                                _lib.stream_of(step.q))
    assert rc == _lib.ASPIRE_ERR_CAPACITY
    assert "ASPIRE_STATIC_SCRATCH_BYTES" in _lib.lib().aspire_last_error().decode()
    small = HolisticAttentionWrapper(torch.empty(1, device=gpu), "NHD", float_workspace_bytes=_lib.STATIC_SCRATCH_BYTES)
    small.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 16, 8, 128, PAGE, causal=True)
    a = _args(small, step, out, lse, small._float_workspace.data_ptr())
    rc = _lib.lib().aspire_attention_run_static(ctypes.byref(small._layout), ctypes.byref(a), _lib.stream_of(step.q))
    assert rc == _lib.ASPIRE_ERR_INVALID
    assert "float_ws must be NULL" in _lib.lib().aspire_last_error().decode()
