"""RoPE, q/k RMSNorm and the fused append on the GPU against the oracle."""

import numpy as np
import pytest
import torch

from aspire_amd.attention.rope import RopeConfig, apply_rope_inplace, qk_norm_rope_update_kv
from aspire_amd.workloads import PAGE, build_step
from helpers import bits, say
from oracle.append import paged_kv_append
from oracle.rope import qk_norm_rope, rope_frequencies, rope_interleaved, token_positions

pytestmark = pytest.mark.gpu


def bf16_close(got: torch.Tensor, ref: torch.Tensor):
    """Within one bf16 rounding step of the reference (relative 2^-8, plus the fp32 work before it)."""
    g, r = got.float().cpu(), ref.float().cpu()
    tol = r.abs() * 2.0 ** -7 + 1e-6
    bad = (g - r).abs() > tol
    assert not bad.any(), f"{int(bad.sum())} of {bad.numel()} values off; worst {float((g - r).abs().max())}"


@pytest.mark.parametrize("llama31", [False, True])
def test_rope_matches_oracle_up_to_long_positions(gpu, llama31):
    say("rope", llama31)
    g = torch.Generator().manual_seed(3)
    T, HQ, HKV = 40, 32, 8
    q = torch.randn(T, HQ, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(T, HKV, 128, generator=g).to(torch.bfloat16)
    indptr = torch.tensor([0, 1, 5, 5, 30, 36], dtype=torch.int32)  # tokens 36..39 belong to no row
    offsets = torch.tensor([0, 131068, 9, 70000, 32767], dtype=torch.int32)
    cfg = RopeConfig(500000.0, 8.0, 1.0, 4.0, 8192) if llama31 else RopeConfig(1e6)
    ll = dict(low_freq_factor=1.0, high_freq_factor=4.0, old_context_len=8192.0) if llama31 else None
    qd, kd = q.to(gpu), k.to(gpu)
    apply_rope_inplace(qd, kd, indptr.to(gpu), offsets.to(gpu), cfg)
    torch.cuda.synchronize()
    f = rope_frequencies(128, cfg.rope_theta, cfg.rope_scale, ll)
    pos = token_positions(indptr.numpy(), offsets.numpy(), T)
    bf16_close(qd, rope_interleaved(q, pos, f))
    bf16_close(kd, rope_interleaved(k, pos, f))
    assert torch.equal(qd[36:].cpu(), q[36:]) and torch.equal(kd[36:].cpu(), k[36:])  # untouched


def test_fused_norm_rope_append_config1_shape(gpu):
    """Qwen3-8B layer: 32 q / 8 kv heads, q/k RMSNorm, permute, rope theta 1e6, append of the 80 new
    tokens into the random-permutation page pool; q rewritten in place, k and v in the cache."""
    say("fused norm+rope+append")
    step = build_step(hq=32, hkv=8, ctx_len=[2000, 40000, 16, 777], q_len=[1, 4, 4, 1], is_draft=[1, 0, 0, 1],
                      draft_budget=64, seed=8, device=gpu, bucket_tokens=12)
    g = torch.Generator().manual_seed(9)
    T = step.total_tokens
    q = torch.randn(12, 32, 128, generator=g).to(torch.bfloat16) * 3   # bucket of 12: 2 padding tokens
    k = torch.randn(12, 8, 128, generator=g).to(torch.bfloat16) * 3
    v = torch.randn(12, 8, 128, generator=g).to(torch.bfloat16)
    wq = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(128, generator=g) + 0.5).to(torch.bfloat16)
    # positions of each row's first new token: its cache length before the append
    offsets = torch.from_numpy(np.append(step.ctx_len - step.q_len, 0).astype(np.int32))
    cache = step.cache.clone()
    before = cache.cpu()
    qd, kd, vd = q.to(gpu), k.to(gpu), v.to(gpu)
    qk_norm_rope_update_kv(qd, kd, vd, wq.to(gpu), wk.to(gpu), 1e-6, step.qo_indptr, offsets.to(gpu), cache,
                           step.kv_indices, step.kv_indptr, step.last_page_len, PAGE, config=RopeConfig(1e6))
    torch.cuda.synchronize()
    ref_q, ref_k = qk_norm_rope(q, k, step.qo_indptr_host.numpy(), offsets.numpy(), theta=1e6, q_weight=wq,
                                k_weight=wk, eps=1e-6)
    bf16_close(qd[:T], ref_q[:T])
    # the cache equals the plain append of the oracle's rotated k and of v (padding tokens skipped)
    ref_bits = paged_kv_append(bits(ref_k), bits(v), step.qo_indptr_host.numpy(), bits(before),
                               step.kv_indices.cpu().numpy(), step.kv_indptr_host.numpy(),
                               step.last_page_len.cpu().numpy(), PAGE)
    ref_cache = torch.from_numpy(ref_bits.view(np.int16)).view(torch.bfloat16)
    got = cache.cpu()
    changed = (ref_cache != before).any(dim=-1)
    assert torch.equal(got[~changed], before[~changed])  # untouched rows unchanged (bitwise)
    assert torch.equal(got[:, 1], ref_cache[:, 1])       # V: exact copy
    bf16_close(got[:, 0][changed[:, 0]], ref_cache[:, 0][changed[:, 0]])
    assert torch.equal(kd.cpu(), k)                       # k itself is not rewritten by the fused op
