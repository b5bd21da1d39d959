"""Token sampling on the HIP path: drop-in for the ``flashinfer.sampling`` functions the
reference calls.

* ``sampling_from_probs(probs, deterministic=True)`` (aspire/engine/runtime.py:312,709,748);
* ``chain_speculative_sampling(draft_probs, draft_token_ids, target_probs, deterministic=True)``
  (aspire/engine/sampling.py:55,84-86).

Both run one kernel of libaspire_hip.so (``aspire_sampling_from_probs``,
``aspire_chain_speculative_sampling``). The uniforms of the draws are a device tensor:
drawn here with ``torch.rand`` from ``generator`` (torch's default CUDA generator when
None, which graph capture supports), or passed in through ``uniforms`` to reproduce a
draw exactly. FlashInfer's own Philox stream is not reproduced, so a given seed samples
different tokens than the reference; the distributions are the same.
"""

from __future__ import annotations

from typing import Optional

import torch

from aspire_amd import _lib


def _uniforms(shape, device, generator, uniforms):
    if uniforms is None:
        return torch.rand(shape, device=device, dtype=torch.float32, generator=generator)
    if uniforms.shape != tuple(shape) or uniforms.dtype != torch.float32 or not uniforms.is_contiguous():
        raise ValueError(f"uniforms must be a contiguous float32 tensor of shape {tuple(shape)}")
    return uniforms


def sampling_from_probs(probs: torch.Tensor, indices: Optional[torch.Tensor] = None, deterministic: bool = True,
                        generator: Optional[torch.Generator] = None, check_nan: bool = False, *,
                        uniforms: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One token per row of ``probs [B, V]`` (fp32): int32 ``[B]``. ``indices`` maps output rows
    to rows of ``probs`` (FlashInfer's batched-probability form); draws are deterministic."""
    _lib.require_cuda(probs, what="sampling_from_probs")
    if probs.dim() != 2 or probs.dtype != torch.float32 or probs.stride(1) != 1:
        raise ValueError("probs must be a 2-D float32 tensor with contiguous rows")
    if check_nan and torch.isnan(probs).any():
        raise ValueError("probs contains NaN")
    if indices is not None:
        probs = probs.index_select(0, indices.to(device=probs.device, dtype=torch.long))
    rows, vocab = probs.shape
    out = torch.empty(rows, dtype=torch.int32, device=probs.device)
    u = _uniforms((rows,), probs.device, generator, uniforms)
    rc = _lib.lib().aspire_sampling_from_probs(_lib.ptr(probs), probs.stride(0), rows, vocab, _lib.ptr(u),
                                               _lib.ptr(out), _lib.stream_of(probs))
    _lib.check(rc, "sampling_from_probs")
    return out


def chain_speculative_sampling(draft_probs: torch.Tensor, draft_token_ids: torch.Tensor, target_probs: torch.Tensor,
                               maybe_output_accepted_token_num: Optional[torch.Tensor] = None,
                               maybe_output_emitted_draft_token_num: Optional[torch.Tensor] = None,
                               deterministic: bool = True, generator: Optional[torch.Generator] = None, *,
                               uniforms: Optional[torch.Tensor] = None):
    """Speculative verification of ``draft_token_ids [B, D]`` drawn from ``draft_probs [B, D, V]``
    against ``target_probs [B, D + 1, V]``. Returns ``(output_token_ids [B, D + 1] int32,
    output_accepted_token_num [B] int32, output_emitted_draft_token_num [B] int32)``; the two
    counts are added in place to the ``maybe_output_*`` tensors when those are given.
    ``uniforms [B, D + 1]``: column i < D decides draft i, column D draws the final token."""
    _lib.require_cuda(draft_probs, draft_token_ids, target_probs, what="chain_speculative_sampling")
    if draft_probs.dim() != 3 or target_probs.dim() != 3 or draft_token_ids.dim() != 2:
        raise ValueError("draft_probs [B, D, V], draft_token_ids [B, D] and target_probs [B, D + 1, V] expected")
    B, D, V = draft_probs.shape
    if target_probs.shape != (B, D + 1, V) or draft_token_ids.shape != (B, D):
        raise ValueError("shapes disagree: target_probs must be [B, D + 1, V], draft_token_ids [B, D]")
    dp = draft_probs.to(torch.float32).contiguous()
    tp = target_probs.to(torch.float32).contiguous()
    ids = draft_token_ids.to(torch.int32).contiguous()
    dev = dp.device
    out = torch.empty(B, D + 1, dtype=torch.int32, device=dev)
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    emitted = torch.empty(B, dtype=torch.int32, device=dev)
    u = _uniforms((B, D + 1), dev, generator, uniforms)
    rc = _lib.lib().aspire_chain_speculative_sampling(_lib.ptr(dp), _lib.ptr(ids), _lib.ptr(tp), B, D, V, _lib.ptr(u),
                                                      _lib.ptr(out), _lib.ptr(acc), _lib.ptr(emitted),
                                                      _lib.stream_of(dp))
    _lib.check(rc, "chain_speculative_sampling")
    if maybe_output_accepted_token_num is not None:
        maybe_output_accepted_token_num.add_(acc)
        acc = maybe_output_accepted_token_num
    if maybe_output_emitted_draft_token_num is not None:
        maybe_output_emitted_draft_token_num.add_(emitted)
        emitted = maybe_output_emitted_draft_token_num
    return out, acc, emitted


__all__ = ["sampling_from_probs", "chain_speculative_sampling"]
