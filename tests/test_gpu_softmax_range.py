"""Online softmax of the mixed attention and prefill kernels when a row's maximum moves by more
than the rescale slack between pages: the keys of every page are scaled per page (rising along
the row, falling along it, or heavy-tailed at random), so scores span hundreds of log2 units and
the running maxima jump late in the row, in split pieces and across the tile lanes. Checked
against the oracle at the attention tolerance, LSE within 2e-3."""

import numpy as np
import pytest
import torch

from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper
from aspire_amd.attention.prefill import BatchPrefillWithPagedKVCacheWrapper
from aspire_amd.workloads import PAGE, build_step
from helpers import attn_close, say
from oracle.attention import paged_attention

pytestmark = pytest.mark.gpu

PROFILES = ["rising", "falling", "heavy_tailed"]


def scaled_cache(step, profile, seed=0):
    """The step's cache with each row's page j of K scaled by s_j, and V by 1/4: these rows'
    softmax is nearly one-hot, so an output is close to a single V value, and at |V| >= 4 one
    bf16 step (1/32) exceeds the absolute tolerance by itself."""
    cache = step.cache.clone()
    cache[:, 1] = (cache[:, 1].float() * 0.25).to(cache.dtype)
    kvp = step.kv_indptr_host.numpy()
    idx = step.kv_indices.cpu().numpy()
    used = idx[: kvp[-1]]
    assert len(np.unique(used)) == len(used), "rows must not share pages"
    rng = np.random.default_rng(seed)
    for b in range(len(kvp) - 1):
        pages = idx[kvp[b] : kvp[b + 1]]
        n = len(pages)
        if profile == "rising":
            s = 1.0 + 0.35 * np.arange(n)
        elif profile == "falling":
            s = 1.0 + 0.35 * np.arange(n)[::-1]
        else:
            s = np.exp(rng.normal(0.0, 1.2, n))
        p = torch.as_tensor(pages, dtype=torch.long, device=cache.device)
        sc = torch.as_tensor(s, dtype=torch.float32, device=cache.device)
        cache[p, 0] = (cache[p, 0].float() * sc[:, None, None, None]).to(cache.dtype)
    return cache


def check(step, cache, out, lse, causal=True):
    ref_out, ref_lse = paged_attention(step.q.cpu(), cache.cpu(), step.qo_indptr_host, step.kv_indptr_host,
                                       step.kv_indices.cpu(), step.kv_len_host, num_kv_heads=step.hkv,
                                       causal=causal)
    T = step.total_tokens
    attn_close(out[:T], ref_out[:T])
    l, rl = lse[:T].cpu(), ref_lse[:T]
    fin = torch.isfinite(rl)
    assert torch.equal(torch.isfinite(l), fin)
    assert (l[fin] - rl[fin]).abs().max().item() < 2e-3


@pytest.mark.parametrize("profile", PROFILES)
@pytest.mark.parametrize("waves_per_cu", [None, 8])
def test_mixed_attention_score_ranges(gpu, profile, waves_per_cu):
    """Drafts over selected pages, verify rows of 1-, 2- and 3-tile items (q_len 3, 5, 9, 12 at
    GQA 4) and rows long enough to be cut into pieces."""
    say("softmax range, mixed attention", profile, waves_per_cu)
    step = build_step(hq=32, hkv=8, ctx_len=[4096 + 5, 3000, 1500, 700, 2500, 333], q_len=[1, 9, 5, 1, 12, 3],
                      is_draft=[1, 0, 0, 1, 0, 0], draft_budget=40, seed=11, device=gpu)
    cache = scaled_cache(step, profile, seed=5)
    kw = {} if waves_per_cu is None else {"waves_per_cu": waves_per_cu}
    w = HolisticAttentionWrapper(torch.empty(1, dtype=torch.uint8, device=gpu), "NHD", **kw)
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, step.hq, step.hkv, 128, PAGE,
           causal=True)
    assert w.plan_info.num_merge > 0  # rows cut into pieces (split-KV)
    out, lse = w.run(step.q, cache, return_lse=True)
    torch.cuda.synchronize()
    check(step, cache, out, lse)


@pytest.mark.parametrize("profile", PROFILES)
def test_prefill_score_ranges(gpu, profile):
    """Causal prompt chunks through the dedicated prefill kernel: a first chunk and a chunk over
    a cached prefix."""
    say("softmax range, prefill", profile)
    step = build_step(hq=32, hkv=8, ctx_len=[2000, 1300], q_len=[2000, 300], is_draft=[0, 0], draft_budget=0,
                      seed=12, device=gpu)
    cache = scaled_cache(step, profile, seed=6)
    w = BatchPrefillWithPagedKVCacheWrapper(torch.empty(1, device=gpu), "NHD")
    w.plan(step.qo_indptr, step.kv_indptr, step.kv_indices, step.last_page_len, 32, 8, 128, PAGE, causal=True)
    assert w._pf is not None
    out, lse = w.run(step.q, cache, return_lse=True)
    torch.cuda.synchronize()
    check(step, cache, out, lse)
