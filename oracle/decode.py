"""The full mixed draft/verify decode step, restated on the CPU (test infrastructure only).

Follows ``TransformerSparseDraft.unified_forward`` (aspire/models/sparse_draft_transformer.py:242-286),
``TransformerBlockSparseDraft.unified_forward`` (:224-239) and
``AttentionSparseDraft.unified_forward`` (:140-177) for one step, with:

* ``RMSNorm`` (transformer.py:505-516) and the residual adds in bf16 (one rounding each);
* linear layers as fp32 products of the bf16 operands rounded once to bf16 (a bf16
  ``nn.Linear`` accumulates in fp32);
* ``FeedForward`` (transformer.py:490-502): ``w2(bf16(silu(w1 x)) * w3 x)``;
* q/k RMSNorm + rotary permute + RoPE (``oracle.rope``), the KV append
  (``oracle.append``) and paged attention (``oracle.attention``);
* the refresh layer: full-context attention with key-mean page scores, top-``budget``
  pages per (row, KV head) with the last ``recent_pages`` forced in
  (``oracle.select.topk_pages_per_head``), and per-head page lists
  (``oracle.page_list.build_head_page_lists``) for the layers after it;
* the greedy pick ``torch.argmax`` of the last branch of unified_forward (:280-281).

The row operations (``add_rms_norm``, ``silu_mul``, ``argmax_rows``) are pinned by
closed forms in ``tests/test_decode_cpu.py``; the composition by the per-layer
components, each pinned on its own. The whole step is checked against the GPU
within bf16 tolerances, since the GEMM summation order differs.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle.append import paged_kv_append
from oracle.attention import paged_attention
from oracle.page_list import build_head_page_lists
from oracle.rope import qk_norm_rope, rms_norm
from oracle.select import topk_pages_per_head

PAGE = 16


def add_rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, delta: torch.Tensor | None = None):
    """Returns ``(x', out)``: ``x' = bf16(x + delta)`` (or ``x``), ``out = RMSNorm(x') * weight``."""
    if delta is not None:
        x = (x.float() + delta.float()).to(x.dtype)
    return x, rms_norm(x, weight, eps)


def silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """``bf16(bf16(silu(g)) * u)`` for ``gate_up = [g | u]`` (transformer.py:498-499)."""
    inter = gate_up.shape[-1] // 2
    g = gate_up[..., :inter].float()
    u = gate_up[..., inter:].float()
    s = (g / (1.0 + torch.exp(-g))).to(gate_up.dtype).float()
    return (s * u).to(gate_up.dtype)


def argmax_rows(logits: torch.Tensor) -> torch.Tensor:
    return torch.argmax(logits.float(), dim=-1)


def linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return (x.float() @ w.float().T).to(x.dtype)


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def decode_step(weights, caches: torch.Tensor, shape, ctx_len, q_len, is_draft, block_table, tokens, *, budget: int,
                refresh_layer: int, recent_pages: int, selected, counts, selection_override=None) -> dict:
    """One step on CPU copies. ``caches`` ([L, P, 2, 16, H_kv, 128] bf16) is updated in place
    by the appends. ``selected`` / ``counts`` ([B, H_kv, budget] physical ids, [B, H_kv]) are
    the draft lists in force before the refresh layer. ``selection_override`` (a pair like
    them) replaces the refresh layer's own selection for the layers after it; the oracle's
    own choice is still returned as ``selected_logical`` / ``selected_counts``."""
    ctx = np.asarray(ctx_len, dtype=np.int64)
    ql = np.asarray(q_len, dtype=np.int64)
    dr = np.asarray(is_draft, dtype=bool)
    table = np.asarray(block_table)
    B, H, D = ctx.shape[0], shape.n_local_heads, shape.head_dim
    T = int(ql.sum())
    n_pages = (ctx + PAGE - 1) // PAGE
    last = (ctx - 1) % PAGE + 1
    qo = np.zeros(B + 1, dtype=np.int64)
    qo[1:] = np.cumsum(ql)
    offsets = ctx - ql
    full_ptr = np.zeros(B + 1, dtype=np.int64)
    full_ptr[1:] = np.cumsum(n_pages)
    full_idx = np.concatenate([table[b, : n_pages[b]] for b in range(B)]).astype(np.int64)
    mode = np.where(dr, 0, 1)

    def head_lists(sel, cnt):
        cap = int(np.maximum(np.asarray(cnt).max(initial=0), n_pages.max())) * B * H
        idx = np.zeros(max(cap, 1), dtype=np.int64)
        ptr = np.zeros(B * H + 1, dtype=np.int64)
        build_head_page_lists(mode, sel, cnt, table, n_pages, idx, ptr)
        seg_pages = np.diff(ptr)
        seg_last = np.repeat(last, H)
        kv_len = np.maximum(seg_pages - 1, 0) * PAGE + np.where(seg_pages > 0, seg_last, 0)
        return torch.from_numpy(idx), torch.from_numpy(ptr), torch.from_numpy(kv_len)

    sel, cnt = np.asarray(selected), np.asarray(counts)
    lists = head_lists(sel, cnt)
    out = {}
    x = weights.tok_embeddings[torch.as_tensor(tokens, dtype=torch.int64)]
    ffn_out = None
    qs, kvs = shape.q_size, shape.kv_size
    for layer, lw in enumerate(weights.layers):
        x, a = add_rms_norm(x, lw["attention_norm"], shape.norm_eps, ffn_out)
        qkv = linear(a, lw["wqkv"])
        q = qkv[:, :qs].reshape(T, shape.n_head, D)
        k = qkv[:, qs : qs + kvs].reshape(T, H, D)
        v = qkv[:, qs + kvs :].reshape(T, H, D)
        q, k = qk_norm_rope(q, k, qo, offsets, theta=shape.rope_base, q_weight=lw["q_norm"],
                            k_weight=lw["k_norm"], eps=shape.norm_eps)
        out[f"q{layer}"] = q
        cache_bits = _bits(caches[layer])
        new = paged_kv_append(_bits(k), _bits(v), qo, cache_bits, full_idx, full_ptr, last, PAGE)
        caches[layer].copy_(torch.from_numpy(new.view(np.int16)).view(torch.bfloat16))
        if layer == refresh_layer:
            scores = torch.zeros(B * H, int(n_pages.max()), dtype=torch.float32)
            y, _ = paged_attention(q, caches[layer], qo, full_ptr, torch.from_numpy(full_idx), ctx, num_kv_heads=H,
                                   page_scores=scores)
            logical, c = topk_pages_per_head(scores, np.repeat(n_pages, H), budget, recent_pages)
            logical = logical.numpy().reshape(B, H, budget)
            c = c.numpy().reshape(B, H)
            phys = np.zeros_like(logical)
            for b in range(B):
                phys[b] = table[b][logical[b]]
                for g in range(H):
                    phys[b, g, c[b, g]:] = 0
            out.update(page_scores=scores, selected_logical=logical, selected_counts=c, selected=phys)
            if selection_override is not None:
                sel, cnt = (np.asarray(t) for t in selection_override)
            else:
                sel, cnt = phys, c
            lists = head_lists(sel, cnt)
        else:
            idx, ptr, kv_len = lists
            y, _ = paged_attention(q, caches[layer], qo, ptr, idx, kv_len, num_kv_heads=H, per_head_lists=True)
        attn_out = linear(y.reshape(T, qs), lw["wo"])
        x, f = add_rms_norm(x, lw["ffn_norm"], shape.norm_eps, attn_out)
        act = silu_mul(linear(f, lw["w13"]))
        ffn_out = linear(act, lw["w2"])
    x, h = add_rms_norm(x, weights.norm, shape.norm_eps, ffn_out)
    logits = linear(h, weights.output)
    out.update(h=h, logits=logits, ids=argmax_rows(logits))
    return out
