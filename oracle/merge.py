"""Split-KV (flash-decode) state merge, restated on the CPU (test infrastructure only).

The merge FlashInfer's persistent kernel applies to its partial-output
workspace (offsets at ``third_party/flashinfer/aspire.patch:81-85,257-273``):
for chunks ``c`` of one (token, head) with normalised partial output ``o_c``
and base-2 log-sum-exp ``lse_c``,

    lse = log2(sum_c 2^lse_c),   o = sum_c 2^(lse_c - lse) * o_c.

Pinned by ``tests/test_oracle_attention.py`` (the merge tests): splitting a row's keys into chunks,
attending each chunk with ``oracle.attention`` and merging reproduces the
unsplit attention (a closed-form identity); merging one chunk is the identity;
a chunk with ``lse = -inf`` contributes nothing.
"""

from __future__ import annotations

import torch


def merge_states(v: torch.Tensor, s: torch.Tensor):
    """Merge ``n`` partial states. ``v``: ``[n, ..., D]``, ``s``: ``[n, ...]`` (base 2)."""
    v = v.float()
    s = s.float()
    m = s.amax(dim=0)
    m_safe = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
    w = torch.exp2(s - m_safe)
    tot = w.sum(dim=0)
    lse = torch.where(tot > 0, m_safe + torch.log2(tot), torch.full_like(tot, float("-inf")))
    wn = w / torch.where(tot > 0, tot, torch.ones_like(tot))
    o = (wn.unsqueeze(-1) * v).sum(dim=0)
    return o, lse
