"""Paged mixed draft/verify attention, restated on the CPU (test infrastructure only).

Semantics of one planned row ``b`` (``aspire/attention/holistic_wrapper.py:344-386``
running FlashInfer's persistent kernel, patched by
``third_party/flashinfer/aspire.patch``):

* queries ``q[qo_indptr[b]:qo_indptr[b+1]]`` (``qo_len`` tokens), keys/values the
  first ``kv_len[b]`` token slots of the pages ``kv_indices[kv_indptr[b]:kv_indptr[b+1]]``
  taken in list order; cache layout ``[P, 2, page, H_kv, D]`` with K at ``[:, 0]``
  and V at ``[:, 1]`` (``aspire/models/mixed_transformer.py:35-40``);
* GQA: q head ``h`` reads kv head ``h // (H_q / H_kv)``;
* causal masking is bottom-right aligned: query ``i`` sees key ``j`` iff
  ``j <= kv_len - qo_len + i`` (every call site passes ``causal=True``,
  ``aspire/backends/base.py:1284,1297``);
* ``p = softmax(q.k * sm_scale)``, ``sm_scale = 1/sqrt(D)`` by default
  (holistic_wrapper.py:359-361); output bf16, ``lse`` in base 2:
  ``lse = log2(sum_j 2^(q.k_j * sm_scale * log2(e)))``;
* the refresh-layer dump (``aspire/backends/jit_kernels.py:182-193,247-256``)
  stores ``fp16(q.k)`` (the raw, unscaled logit) at
  ``dump[((b*num_heads + h)*slots + slot)*kv_stride + j]``; ``first_last`` writes
  query 0 to slot 0 and query ``qo_len-1`` to slot 1, ``last_token`` writes
  query ``qo_len-1`` to its single slot. The dump is taken before the causal
  mask, so masked keys are still dumped. Only ``j < kv_len`` is written.

The per-KV-head page-score epilogue has no reference
counterpart: for a ``qo_len == 1`` row, page ``j`` of kv head ``g`` scores
``max_{h in group(g)} q_h . mean_t(k_{j,t,g})`` over the page's valid keys.

Pinned by ``tests/test_oracle_attention.py``: agreement with
``torch.nn.functional.scaled_dot_product_attention`` on densely gathered K/V
with an explicit bottom-right mask, an fp64 brute-force loop on tiny inputs,
invariance under a permutation of the physical page pool, and the
split + merge identity (see ``oracle.merge``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

LOG2E = 1.4426950408889634


@dataclass
class DumpSpec:
    """Where and how the logits dump is written (the dump JIT variant's parameters)."""

    buffer: torch.Tensor  # flat fp16 (or fp32) tensor, modified in place
    kind: str = "first_last"  # "first_last" (2 slots) or "last_token" (1 slot)
    num_heads: int = 0
    kv_stride: int = 0
    mode_flags: torch.Tensor | None = None  # per row; 0 disables the dump for that row

    @property
    def slots(self) -> int:
        return 2 if self.kind == "first_last" else 1


def _row_kv(cache, kv_indices, start, end, kv_len):
    pages = kv_indices[start:end].long()
    if pages.numel() == 0 or kv_len == 0:
        d = cache.shape[-1]
        h = cache.shape[-2]
        empty = cache.new_zeros((0, h, d))
        return empty, empty
    k = cache[pages, 0].reshape(-1, cache.shape[-2], cache.shape[-1])[:kv_len]
    v = cache[pages, 1].reshape(-1, cache.shape[-2], cache.shape[-1])[:kv_len]
    return k, v


def paged_attention(
    q: torch.Tensor,
    cache: torch.Tensor,
    qo_indptr,
    kv_indptr,
    kv_indices: torch.Tensor,
    kv_len,
    *,
    num_kv_heads: int,
    causal: bool = True,
    sm_scale: float | None = None,
    per_head_lists: bool = False,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    dump: DumpSpec | None = None,
    page_scores: torch.Tensor | None = None,
    compute_dtype: torch.dtype = torch.float32,
):
    """Return ``(out bf16 [T, H_q, D], lse fp32 [T, H_q])`` for every planned row.

    ``per_head_lists``: ``kv_indptr`` has ``B*H_kv + 1`` entries and ``kv_len``
    ``B*H_kv`` entries, one page list per (row, kv head); otherwise one list per row.
    ``page_scores`` (optional, ``[B*H_kv, max_pages]`` fp32) receives the key-mean
    page scores of single-query rows.
    """
    T, hq, d = q.shape
    group = hq // num_kv_heads
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(d)
    qo = [int(x) for x in qo_indptr]
    kvp = [int(x) for x in kv_indptr]
    kvl = [int(x) for x in kv_len]
    bsz = len(kvl) // num_kv_heads if per_head_lists else len(kvl)
    if out is None:
        out = torch.zeros((T, hq, d), dtype=torch.bfloat16)
    if lse is None:
        lse = torch.zeros((T, hq), dtype=torch.float32)
    qf = q.to(compute_dtype)
    for b in range(bsz):
        q0, q1 = qo[b], min(qo[b + 1], T)
        qlen = q1 - q0
        if qlen <= 0:
            continue
        for g in range(num_kv_heads):
            seg = b * num_kv_heads + g if per_head_lists else b
            n = kvl[seg]
            kk, vv = _row_kv(cache, kv_indices, kvp[seg], kvp[seg + 1], n)
            kg = kk[:, g].to(compute_dtype)  # [n, D]
            vg = vv[:, g].to(compute_dtype)
            heads = list(range(g * group, (g + 1) * group))
            qs = qf[q0:q1][:, heads]  # [qlen, G, D]
            s = torch.einsum("igd,jd->gij", qs, kg)  # raw logits [G, qlen, n]
            if dump is not None and n > 0:
                enabled = dump.mode_flags is None or int(dump.mode_flags[b]) != 0
                if enabled:
                    _write_dump(dump, b, heads, s, qlen, n)
            if page_scores is not None and qlen == 1 and n > 0:
                # page j's key mean over its valid keys (the last page may be partial)
                npages = (n + 15) // 16
                padded = torch.cat([kg, kg.new_zeros(npages * 16 - n, d)]) if npages * 16 > n else kg
                count = torch.full((npages, 1), 16.0, dtype=compute_dtype)
                count[-1] = n - (npages - 1) * 16
                kmean = padded.view(npages, 16, d).sum(dim=1) / count
                page_scores[b * num_kv_heads + g, :npages] = (qs[0] @ kmean.T).amax(dim=0).to(page_scores.dtype)
            x = s * (sm_scale * LOG2E)
            if causal and n > 0:
                i_idx = torch.arange(qlen).view(1, qlen, 1)
                j_idx = torch.arange(n).view(1, 1, n)
                x = x.masked_fill(j_idx > (n - qlen + i_idx), float("-inf"))
            if n == 0:
                o = torch.zeros((group, qlen, d), dtype=compute_dtype)
                l = torch.full((group, qlen), float("-inf"), dtype=compute_dtype)
            else:
                m = x.amax(dim=-1, keepdim=True)
                m_safe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
                p = torch.exp2(x - m_safe)
                den = p.sum(dim=-1, keepdim=True)
                o = (p @ vg) / torch.where(den > 0, den, torch.ones_like(den))
                l = torch.where(den > 0, m_safe + torch.log2(den), torch.full_like(den, float("-inf")))[..., 0]
            for gi, h in enumerate(heads):
                out[q0:q1, h] = o[gi].to(out.dtype)
                lse[q0:q1, h] = l[gi].to(lse.dtype)
    return out, lse


def _write_dump(dump: DumpSpec, b: int, heads, s: torch.Tensor, qlen: int, n: int) -> None:
    buf = dump.buffer
    stride = dump.kv_stride
    slots = dump.slots
    targets = []
    if dump.kind == "first_last":
        targets.append((0, 0))
        if qlen > 1:
            targets.append((qlen - 1, 1))
    elif dump.kind == "last_token":
        targets.append((qlen - 1, 0))
    else:
        raise ValueError(f"unknown dump kind {dump.kind!r}")
    for gi, h in enumerate(heads):
        for qi, slot in targets:
            base = ((b * dump.num_heads + h) * slots + slot) * stride
            buf[base : base + n] = s[gi, qi].to(buf.dtype)
