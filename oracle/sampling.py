"""Token sampling and speculative verification, restated on the CPU (test infrastructure only).

The reference samples through FlashInfer (un-vendored, pinned at commit
``56ed54098411946525da17eca2bcfd7ec72a515e``, scripts/install_flashinfer.sh:4-5):

* ``local_topk_candidates`` (aspire/engine/sampling.py:6-29): the ``top_k`` largest
  logits of each row and their vocabulary ids (+ ``vocab_start``), padded with
  ``-inf`` / id 0 when the row is narrower than ``top_k``. ``torch.topk`` leaves the
  order of equal values unspecified; here ties go to the lower id, the order the HIP
  kernel uses.
* ``LogitsPipe([Temperature(), Softmax(), TopP()])`` (aspire/models/
  sparse_draft_runner.py:539-554): ``softmax(values / temperature)`` in fp32, then
  top-p renormalisation: with the probabilities sorted in descending order, the
  smallest prefix whose sum reaches ``top_p`` is kept (with every probability equal to
  the prefix's last one), the rest set to 0, and the kept ones divided by their sum
  (the nucleus of Holtzman et al., 2019).
* ``sampling_from_probs`` (aspire/engine/runtime.py:709,748): inverse-CDF sampling, the
  first index whose inclusive prefix sum exceeds ``u * sum(probs)`` for a uniform
  ``u`` in [0, 1).
* ``chain_speculative_sampling`` (aspire/engine/sampling.py:84-86): speculative
  sampling (Leviathan et al., 2023; Chen et al., 2023). Draft token ``x_i`` with draft
  probability ``q_i(x_i)`` and target probability ``p_i(x_i)`` is accepted when
  ``u_i * q_i(x_i) < p_i(x_i)`` (probability ``min(1, p/q)``); at the first rejection
  ``j`` one token is drawn from ``max(0, p_j - q_j)`` normalised, or, when every draft
  is accepted, from the target's last distribution ``p_D``. Outputs: the accepted
  tokens, the drawn token, then -1; the emitted count ``j``; and the number of
  positions that would be accepted independently of the chain.

FlashInfer draws its uniforms from its own Philox stream, which cannot be reproduced
here; every function takes the uniforms explicitly instead (the HIP kernels do too).
Pinned by closed forms and frequency tests in ``tests/test_oracle_sampling.py``.
"""

from __future__ import annotations

import numpy as np
import torch


def topk_candidates(logits: torch.Tensor, top_k: int, vocab_start: int = 0):
    """``(values [R, top_k], ids [R, top_k] int64)``: descending values, ties to the lower id."""
    if top_k < 1:
        raise ValueError("top_k must be positive")
    R, V = logits.shape
    k = min(top_k, V)
    vals = logits.float().numpy()
    values = torch.full((R, top_k), float("-inf"), dtype=logits.dtype)
    ids = torch.zeros((R, top_k), dtype=torch.int64)
    for r in range(R):
        order = np.lexsort((np.arange(V), -vals[r]))[:k]     # by -value, then by id
        ids[r, :k] = torch.from_numpy(order.astype(np.int64)) + vocab_start
        values[r, :k] = logits[r, torch.from_numpy(order)]
    return values, ids


def logits_pipe(values: torch.Tensor, temperature: float | None = None, top_p: float | None = None):
    """Temperature (skipped when None or <= 0), softmax, top-p (skipped when None, <= 0 or >= 1)."""
    x = values.float()
    if temperature is not None and temperature > 0:
        x = x / temperature
    probs = torch.softmax(x, dim=-1)
    if top_p is None or top_p <= 0 or top_p >= 1:
        return probs
    out = torch.zeros_like(probs)
    for r in range(probs.shape[0]):
        p = probs[r].double()
        srt = torch.sort(p, descending=True).values
        csum = torch.cumsum(srt, dim=0)
        n = int(torch.searchsorted(csum, torch.tensor([top_p], dtype=torch.float64)).item()) + 1
        n = min(n, p.numel())
        thresh = srt[n - 1]
        keep = p >= thresh
        out[r] = torch.where(keep, p / p[keep].sum(), torch.zeros_like(p)).float()
    return out


def cut_margin(probs_row: np.ndarray, top_p: float) -> float:
    """Distance of ``top_p`` from the nearest prefix sum of the descending probabilities: a
    top-p cut closer than rounding can move is ambiguous (tests skip such rows)."""
    csum = np.cumsum(np.sort(probs_row.astype(np.float64))[::-1])
    return float(np.min(np.abs(csum - top_p)))


def sample_from_probs(probs: torch.Tensor, uniforms: torch.Tensor) -> torch.Tensor:
    """``[R]`` int64: first index whose inclusive prefix sum exceeds ``u * sum`` (the last
    positive index when rounding leaves none)."""
    p = probs.double().numpy()
    u = uniforms.double().numpy()
    out = np.zeros(p.shape[0], dtype=np.int64)
    for r in range(p.shape[0]):
        out[r] = _draw(p[r], u[r])
    return torch.from_numpy(out)


def _draw(p: np.ndarray, u: float) -> int:
    csum = np.cumsum(p)
    target = u * csum[-1]
    hit = np.flatnonzero(csum > target)
    if hit.size:
        return int(hit[0])
    pos = np.flatnonzero(p > 0)
    return int(pos[-1]) if pos.size else 0


def draw_margin(p: np.ndarray, u: float) -> float:
    """Relative distance of ``u * sum`` from the nearest prefix sum (ambiguous draws are skipped)."""
    csum = np.cumsum(p.astype(np.float64))
    if csum[-1] <= 0:
        return 0.0
    return float(np.min(np.abs(csum - u * csum[-1])) / csum[-1])


def chain_speculative_sampling(draft_probs: torch.Tensor, draft_token_ids: torch.Tensor, target_probs: torch.Tensor,
                               uniforms: torch.Tensor):
    """``(output [R, D+1] int32, accepted [R] int32, emitted [R] int32)``.

    ``draft_probs [R, D, V]``, ``draft_token_ids [R, D]``, ``target_probs [R, D+1, V]``;
    ``uniforms [R, D+1]``: ``u[:, i]`` decides draft ``i``, ``u[:, D]`` draws the final token."""
    R, D, V = draft_probs.shape
    q = draft_probs.double().numpy()
    p = target_probs.double().numpy()
    x = draft_token_ids.long().numpy()
    u = uniforms.double().numpy()
    out = np.full((R, D + 1), -1, dtype=np.int32)
    accepted = np.zeros(R, dtype=np.int32)
    emitted = np.zeros(R, dtype=np.int32)
    for r in range(R):
        acc = [bool(u[r, i] * q[r, i, x[r, i]] < p[r, i, x[r, i]]) for i in range(D)]
        accepted[r] = sum(acc)
        j = next((i for i in range(D) if not acc[i]), D)
        emitted[r] = j
        out[r, :j] = x[r, :j]
        w = np.maximum(p[r, j] - q[r, j], 0.0) if j < D else p[r, D]
        if w.sum() <= 0:
            w = p[r, j]
        out[r, j] = _draw(w, u[r, D])
    return torch.from_numpy(out), torch.from_numpy(accepted), torch.from_numpy(emitted)


def chain_draw_margin(draft_probs, draft_token_ids, target_probs, uniforms, r: int) -> float:
    """Smallest decision margin of row ``r``: acceptance tests ``|u q - p|`` and the final draw."""
    q = draft_probs[r].double().numpy()
    p = target_probs[r].double().numpy()
    x = draft_token_ids[r].long().numpy()
    u = uniforms[r].double().numpy()
    D = q.shape[0]
    margins = [abs(u[i] * q[i, x[i]] - p[i, x[i]]) for i in range(D)]
    acc = [u[i] * q[i, x[i]] < p[i, x[i]] for i in range(D)]
    j = next((i for i in range(D) if not acc[i]), D)
    w = np.maximum(p[j] - q[j], 0.0) if j < D else p[D]
    if w.sum() <= 0:
        w = p[j]
    margins.append(draw_margin(w, u[D]))
    return float(min(margins))


def verify_topk_speculation(draft_probs, draft_ids, draft_tokens, draft_counts, target_probs, target_ids, uniforms):
    """aspire/engine/sampling.py:46-98 with the chain sampler above (uniforms explicit)."""
    requests, max_draft, top_k = draft_probs.shape
    local_vocab = top_k + 1
    draft_pos = torch.arange(max_draft).unsqueeze(0)
    valid_draft = draft_pos < draft_counts.unsqueeze(1)
    target_pos = torch.arange(max_draft + 1).unsqueeze(0)
    valid_target = target_pos <= draft_counts.unsqueeze(1)
    overlap = target_ids[:, :max_draft].unsqueeze(-1) == draft_ids.unsqueeze(-2)
    mapped = (draft_probs.float().unsqueeze(-2) * overlap.float()).sum(dim=-1)
    mapped[~valid_draft] = 0
    local_draft = torch.zeros(requests, max_draft, local_vocab)
    local_draft[:, :, :top_k] = mapped
    masked_target = target_probs.float().clone()
    masked_target[~valid_target] = 0
    local_target = torch.zeros(requests, max_draft + 1, local_vocab)
    local_target[:, :, :top_k] = masked_target
    match = target_ids[:, :max_draft] == draft_tokens.unsqueeze(-1).long()
    in_target = match.any(dim=-1) & valid_draft
    local_tokens = torch.where(in_target, match.float().argmax(dim=-1), top_k).to(torch.int32)
    draft_self = draft_ids == draft_tokens.unsqueeze(-1).long()
    draft_probability = (draft_probs.float() * draft_self.float()).sum(dim=-1)
    local_draft[:, :, top_k] = draft_probability * (~in_target & valid_draft).float()
    local_draft[~valid_draft, top_k] = 1.0
    out_local, _, emitted = chain_speculative_sampling(local_draft, local_tokens, local_target, uniforms)
    emitted = torch.minimum(emitted, draft_counts.to(emitted.dtype))
    valid = (out_local >= 0) & (out_local < top_k)
    gathered = torch.gather(target_ids, 2, out_local.clamp(0, top_k - 1).long().unsqueeze(-1)).squeeze(-1)
    output = torch.where(valid, gathered, torch.full_like(gathered, -1))
    decode_idx = torch.arange(max_draft + 1).unsqueeze(0)
    output[decode_idx > emitted.unsqueeze(1)] = -1
    return output, emitted, (local_draft, local_tokens, local_target)
