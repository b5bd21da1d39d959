"""QK RMSNorm, the rotary layout permute and interleaved RoPE, restated on the CPU
(test infrastructure only).

Follows the per-layer sequence of the reference's mixed forward
(aspire/models/sparse_draft_transformer.py:149-171):

* ``RMSNorm`` (aspire/models/transformer.py:505-516): ``(x.float() * rsqrt(mean(x^2) + eps))``
  cast back to the input dtype, then multiplied by the weight in that dtype (two bf16
  roundings for a bf16 model);
* ``_permute_for_rope`` (transformer.py:360-364): ``[a_0..a_{D/2-1} | b_0..b_{D/2-1}]`` becomes
  ``[a_0, b_0, a_1, b_1, ...]``;
* ``mylib::rope`` (aspire/models/mixed_transformer.py:159-198): FlashInfer's
  ``apply_rope_inplace`` / ``apply_llama31_rope_inplace`` with ``interleave=True`` —
  pair ``(x_{2i}, x_{2i+1})`` of a token at position ``p`` turns by ``p * f_i``, with
  ``f_i = theta^(-2i/D) / rope_scale``, or the Llama 3.1 smoothing of ``f_i`` between
  ``low_freq_factor`` and ``high_freq_factor`` (the published Llama 3.1 rule). A token
  of row ``b`` sits at ``offsets[b] + (t - indptr[b])``.

FlashInfer (CUDA-only, absent here) evaluates the angle as one fp32 product of the
position and the fp32 frequency and then uses fast fp32 intrinsics; this restatement
keeps the fp32 angle and takes sin / cos of it exactly (fp64), so it is the mathematical
value at the reference's angle precision. The GPU kernel is held to it within one bf16
rounding step.

Pinned by: position 0 is the identity; every pair keeps its norm; the dot product of a
rotated q and k depends only on their position difference; the permute matches its
index definition; RMSNorm of a constant vector is the weight; the Llama 3.1 frequencies
match the published piecewise definition at its three regions
(``tests/test_rope_cpu.py``).
"""

from __future__ import annotations

import math

import numpy as np
import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """transformer.py:505-516 for a bf16 (or any) input: fp32 normalise, cast, scale."""
    xf = x.float()
    out = (xf * torch.rsqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + eps)).to(x.dtype)
    return out * weight.to(x.dtype)


def permute_for_rope(x: torch.Tensor) -> torch.Tensor:
    """``[first half | second half]`` -> interleaved pairs (transformer.py:360-364)."""
    *lead, d = x.shape
    return x.reshape(*lead, 2, d // 2).transpose(-2, -1).reshape(*lead, d)


def rope_frequencies(head_dim: int, theta: float, scale: float = 1.0, llama31: dict | None = None) -> np.ndarray:
    """fp32 frequency of each rotated pair (head_dim / 2 values), correctly rounded."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    base = theta ** (-2.0 * i / head_dim)
    if llama31 is None:
        return (base / scale).astype(np.float32)
    lo_f, hi_f, old = llama31["low_freq_factor"], llama31["high_freq_factor"], llama31["old_context_len"]
    wavelen = 2 * math.pi / base
    low_wavelen, high_wavelen = old / lo_f, old / hi_f
    out = np.empty_like(base)
    for j, (f, w) in enumerate(zip(base, wavelen)):
        if w < high_wavelen:           # high frequency: unchanged
            out[j] = f
        elif w > low_wavelen:          # low frequency: scaled
            out[j] = f / scale
        else:                          # in between: interpolated
            s = (old / w - lo_f) / (hi_f - lo_f)
            out[j] = (1 - s) * f / scale + s * f
    return out.astype(np.float32)


def token_positions(indptr, offsets, total_tokens: int) -> np.ndarray:
    """Position of every token covered by ``indptr``; -1 for tokens outside all rows."""
    ind = np.asarray(indptr, dtype=np.int64)
    off = np.asarray(offsets, dtype=np.int64)
    pos = np.full(total_tokens, -1, dtype=np.int64)
    for b in range(len(ind) - 1):
        for t in range(max(ind[b], 0), min(ind[b + 1], total_tokens)):
            pos[t] = off[b] + (t - ind[b])
    return pos


def rope_interleaved(x: torch.Tensor, pos: np.ndarray, freqs: np.ndarray) -> torch.Tensor:
    """Rotate pairs (2i, 2i+1) of ``x`` [T, H, D] by pos[t] * freqs[i]; tokens with pos < 0 stay."""
    xf = x.double().clone()
    out = xf.clone()
    for t in range(x.shape[0]):
        if pos[t] < 0:
            continue
        ang = (np.float32(pos[t]) * freqs).astype(np.float32).astype(np.float64)  # fp32 angle
        c = torch.from_numpy(np.cos(ang))
        s = torch.from_numpy(np.sin(ang))
        a, b = xf[t, :, 0::2], xf[t, :, 1::2]
        out[t, :, 0::2] = a * c - b * s
        out[t, :, 1::2] = b * c + a * s
    return out.to(x.dtype)


def qk_norm_rope(q, k, indptr, offsets, *, theta, scale=1.0, llama31=None, q_weight=None, k_weight=None,
                 eps=1e-6, permute=True):
    """The reference's per-layer q/k preparation: optional norm + permute, then RoPE."""
    if q_weight is not None:
        q = rms_norm(q, q_weight, eps)
        k = rms_norm(k, k_weight, eps)
        if permute:
            q, k = permute_for_rope(q), permute_for_rope(k)
    freqs = rope_frequencies(q.shape[-1], theta, scale, llama31)
    pos = token_positions(indptr, offsets, q.shape[0])
    return rope_interleaved(q, pos, freqs), rope_interleaved(k, pos, freqs)
