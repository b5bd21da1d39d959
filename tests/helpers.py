"""Shared helpers for the GPU parity tests."""

from __future__ import annotations

import sys

import numpy as np
import torch

from aspire_amd.workloads import PAGE, MixedStep


def say(*msg):
    """Name the case before a GPU step (flushed, so a failing box still shows it)."""
    print("[case]", *msg, file=sys.stderr, flush=True)


def bits(t: torch.Tensor) -> np.ndarray:
    """uint16 bit pattern of a 16-bit tensor, on the host."""
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def attn_close(out: torch.Tensor, ref: torch.Tensor, max_abs=2e-2, mean_abs=2e-3):
    """BASELINE tolerance for bf16 attention output with fp32 accumulation."""
    d = (out.float().cpu() - ref.float().cpu()).abs()
    assert torch.isfinite(out.float()).all(), "non-finite output"
    assert d.max().item() <= max_abs, f"max abs {d.max().item():.4g} > {max_abs}"
    assert d.mean().item() <= mean_abs, f"mean abs {d.mean().item():.4g} > {mean_abs}"


def rows_tokens(step: MixedStep):
    qo = step.qo_indptr_host.numpy()
    return [(b, int(qo[b]), int(qo[b + 1])) for b in range(step.batch)]


def oracle_append(step: MixedStep, cache_bits: np.ndarray) -> np.ndarray:
    from oracle.append import paged_kv_append

    return paged_kv_append(
        bits(step.k_new), bits(step.v_new), step.qo_indptr_host.numpy(), cache_bits,
        step.kv_indices.cpu().numpy(), step.kv_indptr_host.numpy(), step.last_page_len.cpu().numpy(), PAGE)


def assert_topk_sets(selected_logical, scores, k, tol=1e-3):
    """Selected set equals the top-k of ``scores`` wherever the score gap exceeds ``tol``."""
    got = set(int(x) for x in selected_logical)
    assert len(got) == k, f"selected {len(got)} pages, expected {k}"
    if k == 0:
        return
    s = np.asarray(scores, dtype=np.float64)
    t = np.sort(s)[::-1][k - 1]
    must = set(np.flatnonzero(s > t + tol).tolist()) if np.isfinite(t) else set(np.flatnonzero(s > t).tolist())
    must_not = set(np.flatnonzero(s < t - tol).tolist()) if np.isfinite(t) else set(np.flatnonzero(s < t).tolist())
    assert must <= got, f"missing pages {sorted(must - got)[:10]}"
    assert not (got & must_not), f"extra pages {sorted(got & must_not)[:10]}"


def oracle_row(q: torch.Tensor, cache: torch.Tensor, tokens, page_lists, kv_lens, num_kv_heads: int,
               per_head: bool = False, **kw):
    """CPU oracle for one row whose pages are gathered on the device first (only the row's
    pages cross to the host). ``page_lists``: the row's physical page list, or with
    ``per_head`` one list per kv head (``kv_lens`` then per head); ``tokens``: the row's token
    indices into ``q``. Returns ``(out [t, H_q, D], lse [t, H_q])``; extra keywords go to the
    oracle."""
    from oracle.attention import paged_attention

    lists = [torch.as_tensor(np.asarray(p), dtype=torch.int64) for p in (page_lists if per_head else [page_lists])]
    used = torch.cat(lists)
    uniq, inv = torch.unique(used, return_inverse=True)
    small = cache[uniq.to(cache.device)].cpu()
    kvp = np.concatenate([[0], np.cumsum([len(x) for x in lists])])
    toks = list(tokens)
    return paged_attention(q[toks].cpu(), small, [0, len(toks)], kvp, inv.to(torch.int32),
                           [int(x) for x in kv_lens], num_kv_heads=num_kv_heads, per_head_lists=per_head, **kw)
