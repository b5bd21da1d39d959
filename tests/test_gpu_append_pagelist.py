"""KV append and mixed page list on the GPU: bit-exact against the oracle."""

import numpy as np
import pytest
import torch

import aspire_amd.attention.kv_ops  # noqa: F401  (registers mylib ops)
from aspire_amd.attention.page_list import build_unified_indices
from aspire_amd.workloads import PAGE, build_step, config0, config1
from helpers import bits, oracle_append, say
from oracle.append import paged_kv_append
from oracle.page_list import build_unified_indices as oracle_build

pytestmark = pytest.mark.gpu


def _append(step, cache):
    torch.ops.mylib.update_kv_padded(step.k_new, step.v_new, step.qo_indptr, cache, step.kv_indices,
                                     step.kv_indptr, step.last_page_len, PAGE)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_append_random_ragged_matches_oracle(gpu, seed):
    rng = np.random.default_rng(seed)
    B = int(rng.integers(1, 9))
    ctx = rng.integers(1, 300, size=B)
    qlen = np.minimum(rng.integers(1, 6, size=B), ctx)
    draft = rng.random(B) < 0.5
    say("append random", seed, B, ctx.tolist(), qlen.tolist())
    step = build_step(hq=8, hkv=4, ctx_len=ctx, q_len=qlen, is_draft=draft, draft_budget=3,
                      pool_pages=int(((ctx + 15) // 16).sum()) + 5, seed=seed, device=gpu,
                      bucket_tokens=int(qlen.sum()) + 3)
    # pad the new-token tensors to the bucket: padding tokens must be skipped
    T = int(step.qo_indptr_host[-1])
    pad = T - step.total_tokens
    step.k_new = torch.cat([step.k_new, torch.randn(pad, 4, 128, device=gpu).bfloat16()])
    step.v_new = torch.cat([step.v_new, torch.randn(pad, 4, 128, device=gpu).bfloat16()])
    raw = torch.randint(-32768, 32767, step.cache.shape, dtype=torch.int16, device=gpu)
    cache = raw.view(torch.bfloat16).clone()
    before = bits(cache)
    _append(step, cache)
    torch.cuda.synchronize()
    assert np.array_equal(bits(cache), oracle_append(step, before))


def test_append_config0_and_strided_tokens(gpu):
    say("append config0 strided")
    step = config0(device=gpu)
    before = bits(step.cache)
    expect = oracle_append(step, before)
    # k/v as column slices of a fused qkv projection (token stride > heads * head_dim)
    T = step.k_new.shape[0]
    fused = torch.randn(T, 16 * 128 + 2 * 8 * 128, device=gpu).bfloat16()
    fused[:, 16 * 128 : 24 * 128] = step.k_new.reshape(T, -1)
    fused[:, 24 * 128 :] = step.v_new.reshape(T, -1)
    k = fused[:, 16 * 128 : 24 * 128].view(T, 8, 128)
    v = fused[:, 24 * 128 :].view(T, 8, 128)
    assert k.stride(0) == 32 * 128
    cache = step.cache.clone()
    torch.ops.mylib.update_kv_padded(k, v, step.qo_indptr, cache, step.kv_indices, step.kv_indptr,
                                     step.last_page_len, PAGE)
    torch.cuda.synchronize()
    assert np.array_equal(bits(cache), expect)
    # update_kv (unpadded op) shares the kernel
    cache2 = step.cache.clone()
    torch.ops.mylib.update_kv(step.k_new, step.v_new, step.qo_indptr, cache2, step.kv_indices, step.kv_indptr,
                              step.last_page_len, PAGE)
    torch.cuda.synchronize()
    assert np.array_equal(bits(cache2), expect)


def test_append_rejects_noncontiguous_heads(gpu):
    step = config0(device=gpu)
    k = step.k_new.transpose(0, 1).contiguous().transpose(0, 1)
    with pytest.raises(ValueError, match="contiguous k/v heads"):
        torch.ops.mylib.update_kv_padded(k, step.v_new, step.qo_indptr, step.cache, step.kv_indices,
                                         step.kv_indptr, step.last_page_len, PAGE)


def test_append_full_size_config1_roundtrip(gpu):
    say("append config1 full size")
    step = config1(device=gpu)
    cache = step.cache
    before = cache.clone()
    _append(step, cache)
    torch.cuda.synchronize()
    # round trip: every new token is found at its (page, slot)
    qo = step.qo_indptr_host.numpy()
    kvp = step.kv_indptr_host.numpy()
    idx = step.kv_indices.cpu().numpy()
    kvl = step.kv_len_host.numpy()
    pages, slots, toks = [], [], []
    for b in range(step.batch):
        for i in range(qo[b], qo[b + 1]):
            pos = kvl[b] - (qo[b + 1] - i)
            pages.append(idx[kvp[b] + pos // PAGE])
            slots.append(pos % PAGE)
            toks.append(i)
    pg = torch.tensor(pages, device=gpu).long()
    sl = torch.tensor(slots, device=gpu).long()
    tk = torch.tensor(toks, device=gpu).long()
    assert torch.equal(cache[pg, 0, sl], step.k_new[tk])
    assert torch.equal(cache[pg, 1, sl], step.v_new[tk])
    # nothing else changed
    changed = (cache.view(torch.int16) != before.view(torch.int16)).any(dim=-1).any(dim=-1)  # [P, 2, 16]
    written = torch.zeros_like(changed)
    written[pg, :, sl] = True
    assert not (changed & ~written).any()


@pytest.mark.parametrize("mode_dtype", [torch.int32, torch.int64, torch.bool])
def test_page_list_matches_oracle(gpu, mode_dtype):
    rng = np.random.default_rng(7)
    B, dw, vw = 37, 9, 300
    say("page list", mode_dtype)
    mode = rng.integers(0, 2, size=B)
    draft = rng.integers(0, 10000, size=(B, dw)).astype(np.int32)
    verify = rng.integers(0, 10000, size=(B, vw)).astype(np.int32)
    dn = rng.integers(0, dw + 1, size=B).astype(np.int32)
    vn = rng.integers(0, vw + 1, size=B).astype(np.int32)
    cap = B * vw
    idx_ref = np.full(cap, -5, dtype=np.int32)
    ptr_ref = np.full(B + 3, -9, dtype=np.int32)
    oracle_build(mode, draft, verify, dn, vn, idx_ref, ptr_ref)
    dev = lambda a: torch.from_numpy(a).to(gpu)
    flags = dev(mode.astype(np.int64)).to(mode_dtype)
    idx = torch.full((cap,), -5, dtype=torch.int32, device=gpu)
    ptr = torch.full((B + 3,), -9, dtype=torch.int32, device=gpu)
    build_unified_indices(flags, dev(draft), dev(verify), dev(dn), dev(vn), idx, ptr)
    torch.cuda.synchronize()
    assert np.array_equal(ptr.cpu().numpy(), ptr_ref)
    assert np.array_equal(idx.cpu().numpy(), idx_ref)
    # padding-row fill variant
    build_unified_indices(flags, dev(draft), dev(verify), dev(dn), dev(vn), idx, ptr, indptr_fill_to=B + 3)
    torch.cuda.synchronize()
    assert (ptr.cpu().numpy()[B + 1 :] == ptr_ref[B]).all()


def test_page_list_builds_config0_mixed_list(gpu):
    step = config0(device=gpu)
    B = step.batch
    width = step.block_table.shape[1]
    draft_tab = torch.zeros(B, 64, dtype=torch.int32, device=gpu)
    dn = torch.zeros(B, dtype=torch.int32, device=gpu)
    for b in range(B):
        if step.draft_pages[b] is not None:
            phys = step.block_table[b, torch.from_numpy(step.draft_pages[b]).to(gpu)]
            draft_tab[b, : phys.numel()] = phys
            dn[b] = phys.numel()
    vn = torch.full((B,), width, dtype=torch.int32, device=gpu)
    idx = torch.zeros(B * width, dtype=torch.int32, device=gpu)
    ptr = torch.zeros(B + 2, dtype=torch.int32, device=gpu)
    build_unified_indices(step.mode_flags, draft_tab, step.block_table, dn, vn, idx, ptr, indptr_fill_to=B + 2)
    torch.cuda.synchronize()
    assert torch.equal(ptr, step.kv_indptr)
    n = int(step.kv_indptr_host[B])
    assert torch.equal(idx[:n], step.kv_indices)
