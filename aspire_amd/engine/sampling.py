"""Sampling helpers of the decode loop on the HIP path: drop-in for
``aspire/engine/sampling.py`` (same names, signatures and outputs).

* ``local_topk_candidates`` (sampling.py:6-29): one ``aspire_topk_candidates`` launch per
  call: the ``top_k`` largest logits of each row, descending, ids offset by ``vocab_start``,
  padded with ``-inf`` / id 0 when the shard is narrower than ``top_k``. Equal logits are
  ordered by the lower id (``torch.topk`` leaves their order unspecified).
* ``merge_topk_candidates`` (sampling.py:32-43): the same kernel over the concatenated
  candidates of the ranks, then a gather of their ids.
* ``verify_topk_speculation`` (sampling.py:46-98): one ``aspire_verify_topk_speculation``
  launch builds each position's local vocabulary (the target's top_k candidates plus one
  entry for any other token) and runs the chain rule over it; ``uniforms`` (optional,
  ``[requests, max_draft + 1]``) fixes the draws.
* ``first_eos`` (sampling.py:101-116): torch ops (a handful of elementwise steps).
"""

from __future__ import annotations

from typing import Optional

import torch

from aspire_amd import _lib


def local_topk_candidates(logits: torch.Tensor, top_k: int, vocab_start: int = 0):
    """``(values [.., top_k] logits dtype, indices [.., top_k] int64)`` of each row's best logits."""
    if top_k < 1:
        raise ValueError("top_k must be positive")
    if logits.shape[-1] < 1:
        raise ValueError("logit shard must contain at least one vocabulary entry")
    _lib.require_cuda(logits, what="local_topk_candidates")
    if logits.dtype != torch.bfloat16:
        raise ValueError("the HIP top-k kernel reads bf16 logits")
    lead = logits.shape[:-1]
    x = logits.reshape(-1, logits.shape[-1])
    if x.stride(-1) != 1:
        x = x.contiguous()
    rows, vocab = x.shape
    values = torch.empty(rows, top_k, dtype=logits.dtype, device=logits.device)
    ids = torch.empty(rows, top_k, dtype=torch.int64, device=logits.device)
    rc = _lib.lib().aspire_topk_candidates(_lib.ptr(x), x.stride(0), rows, vocab, top_k, int(vocab_start),
                                           _lib.ptr(values), _lib.ptr(ids), _lib.stream_of(logits))
    _lib.check(rc, "local_topk_candidates")
    return values.view(*lead, top_k), ids.view(*lead, top_k)


def merge_topk_candidates(values: torch.Tensor, indices: torch.Tensor, top_k: int):
    """Global top-k of rank-local candidates laid side by side (``[.., ranks * k]``)."""
    if values.shape != indices.shape:
        raise ValueError("candidate values and indices must have identical shapes")
    if top_k < 1 or top_k > values.shape[-1]:
        raise ValueError("top_k must fit within the candidate width")
    best, pos = local_topk_candidates(values, top_k)
    return best, torch.gather(indices, -1, pos)


def verify_topk_speculation(draft_probs: torch.Tensor, draft_ids: torch.Tensor, draft_tokens: torch.Tensor,
                            draft_counts: torch.Tensor, target_probs: torch.Tensor, target_ids: torch.Tensor, *,
                            uniforms: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None):
    """``(output [requests, max_draft + 1] int64, emitted [requests] int32)``: the verified tokens
    (vocabulary ids; -1 past the last emitted one) and the accepted draft count per request.

    ``draft_probs`` / ``draft_ids`` ``[requests, max_draft, top_k]`` are each draft position's
    candidate distribution, ``draft_tokens [requests, max_draft]`` the proposed tokens,
    ``draft_counts [requests]`` the valid draft positions, ``target_probs`` / ``target_ids``
    ``[requests, max_draft + 1, top_k]`` the target's candidate distributions."""
    _lib.require_cuda(draft_probs, draft_ids, draft_tokens, draft_counts, target_probs, target_ids,
                      what="verify_topk_speculation")
    requests, max_draft, top_k = draft_probs.shape
    if draft_ids.shape != draft_probs.shape or draft_tokens.shape != (requests, max_draft):
        raise ValueError("draft_ids must match draft_probs and draft_tokens be [requests, max_draft]")
    if target_probs.shape != (requests, max_draft + 1, top_k) or target_ids.shape != target_probs.shape:
        raise ValueError("target_probs / target_ids must be [requests, max_draft + 1, top_k]")
    if draft_counts.shape != (requests,):
        raise ValueError("draft_counts must hold one count per request")
    dev = draft_probs.device
    dp = draft_probs.to(torch.float32).contiguous()
    tp = target_probs.to(torch.float32).contiguous()
    di = draft_ids.to(torch.int64).contiguous()
    ti = target_ids.to(torch.int64).contiguous()
    tok = draft_tokens.to(torch.int32).contiguous()
    cnt = draft_counts.to(torch.int32).contiguous()
    if uniforms is None:
        uniforms = torch.rand(requests, max_draft + 1, device=dev, generator=generator)
    elif uniforms.shape != (requests, max_draft + 1) or uniforms.dtype != torch.float32:
        raise ValueError("uniforms must be float32 [requests, max_draft + 1]")
    u = uniforms.contiguous()
    output = torch.empty(requests, max_draft + 1, dtype=torch.int64, device=dev)
    emitted = torch.empty(requests, dtype=torch.int32, device=dev)
    rc = _lib.lib().aspire_verify_topk_speculation(_lib.ptr(dp), _lib.ptr(di), _lib.ptr(tok), _lib.ptr(cnt),
                                                   _lib.ptr(tp), _lib.ptr(ti), _lib.ptr(u), requests, max_draft,
                                                   top_k, _lib.ptr(output), _lib.ptr(emitted), _lib.stream_of(dp))
    _lib.check(rc, "verify_topk_speculation")
    return output, emitted


def first_eos(output: torch.Tensor, committed: torch.Tensor, eos_token_ids: tuple[int, ...]):
    """Cut each row's ``committed`` tokens after its first end-of-sequence token: returns
    ``(committed', found)`` with committed' = index of the first EOS + 1 where one occurs
    among the committed tokens, else unchanged."""
    found = torch.zeros(output.shape[0], dtype=torch.bool, device=output.device)
    if not eos_token_ids:
        return committed, found
    cols = torch.arange(output.shape[1], device=output.device)
    in_range = cols[None, :] < committed[:, None]
    is_eos = torch.isin(output, torch.tensor(eos_token_ids, device=output.device, dtype=output.dtype)) & in_range
    found = is_eos.any(dim=1)
    # first EOS column: the smallest column index among the EOS hits
    first = torch.where(is_eos, cols[None, :].expand_as(is_eos), output.shape[1]).amin(dim=1).to(torch.int32)
    return torch.where(found, first + 1, committed), found


__all__ = ["local_topk_candidates", "merge_topk_candidates", "verify_topk_speculation", "first_eos"]
