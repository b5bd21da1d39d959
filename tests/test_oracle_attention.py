"""The CPU attention/merge oracles against a library routine, brute force and identities."""

import math

import torch
import torch.nn.functional as F

from oracle.attention import DumpSpec, paged_attention
from oracle.merge import merge_states


def _setup(seed=0, B=3, hq=8, hkv=2, D=16, page=16, lens=(40, 17, 64), qlens=(1, 3, 5), P=20):
    g = torch.Generator().manual_seed(seed)
    npages = [(n + page - 1) // page for n in lens]
    perm = torch.randperm(P, generator=g)
    kv_indptr = [0]
    for n in npages:
        kv_indptr.append(kv_indptr[-1] + n)
    kv_indices = perm[: kv_indptr[-1]].to(torch.int32)
    qo = [0]
    for n in qlens:
        qo.append(qo[-1] + n)
    q = torch.randn(qo[-1], hq, D, generator=g).to(torch.bfloat16)
    cache = torch.randn(P, 2, page, hkv, D, generator=g).to(torch.bfloat16)
    return q, cache, qo, kv_indptr, kv_indices, list(lens)


def test_matches_sdpa_with_bottom_right_mask():
    q, cache, qo, kvp, kvi, lens = _setup()
    hq, hkv, D = q.shape[1], cache.shape[3], q.shape[2]
    out, lse = paged_attention(q, cache, qo, kvp, kvi, lens, num_kv_heads=hkv)
    for b in range(len(lens)):
        pages = kvi[kvp[b]:kvp[b + 1]].long()
        k = cache[pages, 0].reshape(-1, hkv, D)[: lens[b]].float()
        v = cache[pages, 1].reshape(-1, hkv, D)[: lens[b]].float()
        qq = q[qo[b]:qo[b + 1]].float()
        n, m = lens[b], qq.shape[0]
        k = k.repeat_interleave(hq // hkv, dim=1).transpose(0, 1)
        v = v.repeat_interleave(hq // hkv, dim=1).transpose(0, 1)
        mask = torch.arange(n)[None, :] <= (n - m + torch.arange(m))[:, None]
        ref = F.scaled_dot_product_attention(qq.transpose(0, 1), k, v, attn_mask=mask)
        assert torch.allclose(out[qo[b]:qo[b + 1]].float(), ref.transpose(0, 1), atol=1e-2, rtol=0)
        s = (qq.transpose(0, 1) @ k.transpose(1, 2)) / math.sqrt(D)
        s = s.masked_fill(~mask, float("-inf"))
        ref_lse = torch.logsumexp(s, dim=-1) / math.log(2)
        assert torch.allclose(lse[qo[b]:qo[b + 1]], ref_lse.transpose(0, 1), atol=1e-4)


def test_brute_force_fp64_tiny():
    q, cache, qo, kvp, kvi, lens = _setup(seed=1, B=2, hq=4, hkv=2, D=8, lens=(5, 19), qlens=(2, 1))
    out, lse = paged_attention(q, cache, qo, kvp, kvi, lens, num_kv_heads=2, compute_dtype=torch.float64)
    for b in range(2):
        for i in range(qo[b + 1] - qo[b]):
            for h in range(4):
                g = h // 2
                n = lens[b]
                qlen = qo[b + 1] - qo[b]
                num = [0.0] * 8
                den = 0.0
                logits = []
                for j in range(n):
                    if j > n - qlen + i:
                        continue
                    page = int(kvi[kvp[b] + j // 16])
                    kv = cache[page, :, j % 16, g].double()
                    logits.append((j, float((q[qo[b] + i, h].double() * kv[0]).sum()) / math.sqrt(8)))
                mx = max(x for _, x in logits)
                for j, x in logits:
                    page = int(kvi[kvp[b] + j // 16])
                    w = math.exp(x - mx)
                    den += w
                    vv = cache[page, 1, j % 16, g].double()
                    num = [a + w * float(c) for a, c in zip(num, vv)]
                ref = torch.tensor([a / den for a in num], dtype=torch.float64)
                assert torch.allclose(out[qo[b] + i, h].double(), ref, atol=8e-3)
                assert abs(float(lse[qo[b] + i, h]) - (mx + math.log(den)) / math.log(2)) < 1e-6


def test_page_pool_permutation_invariance():
    q, cache, qo, kvp, kvi, lens = _setup(seed=2)
    out1, lse1 = paged_attention(q, cache, qo, kvp, kvi, lens, num_kv_heads=2)
    perm = torch.randperm(cache.shape[0], generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    cache2 = cache[perm]  # new page x holds old page perm[x]
    kvi2 = inv[kvi.long()].to(torch.int32)
    out2, lse2 = paged_attention(q, cache2, qo, kvp, kvi2, lens, num_kv_heads=2)
    assert torch.equal(out1, out2) and torch.equal(lse1, lse2)


def test_split_and_merge_equals_unsplit():
    q, cache, qo, kvp, kvi, lens = _setup(seed=3, lens=(64, 48, 80), qlens=(1, 1, 1))
    full, full_lse = paged_attention(q, cache, qo, kvp, kvi, lens, num_kv_heads=2, causal=False)
    # chunk 0 = first page of each row, chunk 1 = the rest
    parts_o, parts_l = [], []
    for first in (True, False):
        kvp_c, kvl_c, idx = [0], [], []
        for b in range(3):
            pages = kvi[kvp[b]:kvp[b + 1]].tolist()
            sel = pages[:1] if first else pages[1:]
            idx += sel
            kvp_c.append(kvp_c[-1] + len(sel))
            kvl_c.append(16 if first else lens[b] - 16)
        o, l = paged_attention(q, cache, qo, kvp_c, torch.tensor(idx, dtype=torch.int32), kvl_c,
                               num_kv_heads=2, causal=False, out=torch.zeros(q.shape, dtype=torch.float32))
        parts_o.append(o)
        parts_l.append(l)
    mo, ml = merge_states(torch.stack(parts_o), torch.stack(parts_l))
    assert torch.allclose(mo, full.float(), atol=1e-2)
    assert torch.allclose(ml, full_lse, atol=1e-5)


def test_merge_identities():
    v = torch.randn(1, 5, 3, 8)
    s = torch.randn(1, 5, 3)
    o, l = merge_states(v, s)
    assert torch.allclose(o, v[0]) and torch.allclose(l, s[0])
    v2 = torch.cat([v, torch.randn(1, 5, 3, 8)])
    s2 = torch.cat([s, torch.full((1, 5, 3), float("-inf"))])
    o2, l2 = merge_states(v2, s2)
    assert torch.allclose(o2, v[0]) and torch.allclose(l2, s[0])


def test_dump_layout_first_last():
    q, cache, qo, kvp, kvi, lens = _setup(seed=4, lens=(40, 17, 64), qlens=(1, 3, 5))
    stride = 80
    buf = torch.full((3 * 8 * 2 * stride,), float("-inf"), dtype=torch.float16)
    paged_attention(q, cache, qo, kvp, kvi, lens, num_kv_heads=2,
                    dump=DumpSpec(buffer=buf, kind="first_last", num_heads=8, kv_stride=stride))
    view = buf.view(3, 8, 2, stride)
    # row 1 (3 queries), head 5 (kv head 1), slot 1 = last query, key 10
    b, h, j = 1, 5, 10
    page = int(kvi[kvp[b] + j // 16])
    raw = float((q[qo[b] + 2, h].float() * cache[page, 0, j % 16, 1].float()).sum())
    assert abs(float(view[b, h, 1, j]) - raw) <= abs(raw) * 1e-3 + 1e-3
    # masked key of query 0 is still dumped; nothing past kv_len is written
    assert torch.isfinite(view[b, h, 0, : lens[b]]).all()
    assert torch.isinf(view[b, :, :, lens[b]:]).all()
    # single-query row writes slot 0 only
    assert torch.isinf(view[0, :, 1]).all()


def test_keymean_page_scores_closed_forms():
    """The key-mean page score of a single-query row: with every valid key of page j equal
    to c_j the score is max_h q_h . c_j; a partial last page averages only its valid keys
    (the slots past kv_len hold large values that would show if they were counted); rows
    with more than one query leave their scores untouched."""
    g = torch.Generator().manual_seed(8)
    D, hq, hkv, page = 16, 4, 2, 16
    lens = [16 * 3 + 5, 32, 20]          # row 0: partial last page of 5 keys; row 2 has 3 queries
    qlens = [1, 1, 3]
    P = 10
    cache = torch.zeros(P, 2, page, hkv, D, dtype=torch.bfloat16)
    consts = torch.randn(P, hkv, D, generator=g).to(torch.bfloat16)
    cache[:, 0] = consts[:, None]
    pages = [[3, 7, 1, 5], [0, 9], [2, 4]]
    # row 0's last page (5): 5 distinct valid keys, large values in the 11 slots past kv_len
    valid = torch.randn(5, hkv, D, generator=g).to(torch.bfloat16)
    cache[5, 0, :5] = valid
    cache[5, 0, 5:] = 1000.0
    kvp = [0, 4, 6, 8]
    kvi = torch.tensor(sum(pages, []), dtype=torch.int32)
    qo = [0, 1, 2, 5]
    q = torch.randn(5, hq, D, generator=g).to(torch.bfloat16)
    scores = torch.full((3 * hkv, 8), float("nan"))
    paged_attention(q, cache, qo, kvp, kvi, lens, num_kv_heads=hkv, page_scores=scores)
    group = hq // hkv
    for b in (0, 1):
        for kvh in range(hkv):
            qh = q[qo[b], kvh * group : (kvh + 1) * group].double()
            for j, p in enumerate(pages[b]):
                if b == 0 and j == 3:
                    c = valid[:, kvh].double().mean(dim=0)       # only the 5 valid keys
                else:
                    c = consts[p, kvh].double()
                want = float((qh @ c).max())
                assert abs(float(scores[b * hkv + kvh, j]) - want) <= 1e-4 * (1 + abs(want)), (b, kvh, j)
            assert torch.isnan(scores[b * hkv + kvh, len(pages[b]):]).all()
    assert torch.isnan(scores[2 * hkv :]).all()          # 3 queries: no scores
