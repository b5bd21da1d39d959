"""Rotary embedding and the fused q / k preparation of the mixed forward (HIP).

* ``define_rope_op(...)`` registers ``mylib::rope(Tensor(a!) q, Tensor(b!) k, Tensor indptr,
  Tensor offsets) -> ()`` exactly as the reference's ``setup_caches`` does
  (aspire/models/mixed_transformer.py:159-198): FlashInfer's ``apply_rope_inplace`` or,
  with the Llama 3.1 factors, ``apply_llama31_rope_inplace``, both with
  ``interleave=True``; token ``t`` of row ``b`` sits at ``offsets[b] + t - indptr[b]``.
* ``qk_norm_rope_update_kv(...)`` (torch op ``mylib::qk_norm_rope_update_kv``) runs the
  whole per-layer sequence of the mixed forward (sparse_draft_transformer.py:149-171) in
  one launch: q / k RMSNorm, the rotary permute, RoPE, and ``update_kv_padded`` of the
  rotated k and of v; q is rewritten in place (interleaved layout, as the reference's q
  after its permute and rope).

One kernel (``aspire_qk_norm_rope_append``) serves both; head_dim 128, bf16.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from aspire_amd import _lib


@dataclass
class RopeConfig:
    rope_theta: float = 10000.0
    rope_scale: float = 1.0
    low_freq_factor: float | None = None
    high_freq_factor: float | None = None
    original_max_position_embeddings: int | None = None

    @property
    def llama31(self) -> bool:
        return self.low_freq_factor is not None and self.high_freq_factor is not None


_CONFIG = RopeConfig()


def rope_frequencies(head_dim: int = 128, config: RopeConfig | None = None) -> torch.Tensor:
    """The fp32 rotary frequencies the kernel uses (computed on the host)."""
    c = config or _CONFIG
    out = torch.empty(head_dim // 2, dtype=torch.float32)
    _lib.check(_lib.lib().aspire_rope_frequencies(head_dim, c.rope_theta, c.rope_scale, int(c.llama31),
                                                  float(c.low_freq_factor or 0), float(c.high_freq_factor or 0),
                                                  float(c.original_max_position_embeddings or 0),
                                                  ctypes.c_void_p(out.data_ptr())), "rope_frequencies")
    return out


def _i32(t):
    return t if t.dtype == torch.int32 and t.is_contiguous() else t.to(torch.int32).contiguous()


def _run(q, k, indptr, offsets, *, config, v=None, q_norm_weight=None, k_norm_weight=None, eps=1e-6,
         permute=True, kv_cache=None, kv_page_indices=None, kv_page_indptr=None, kv_last_page_len=None,
         page_size=16, write_k=True, what="rope"):
    T = q.shape[0]
    if T == 0:
        return
    _lib.require_cuda(q, k, indptr, offsets, what=what)
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t is not None and (t.dtype != torch.bfloat16 or t.dim() != 3 or t.shape[-1] != 128 or t.stride(-1) != 1):
            raise ValueError(f"{what}: {name} must be bf16 [T, H, 128] with contiguous head dims")
    if k.shape[0] != T or (v is not None and v.shape[0] != T):
        raise ValueError(f"{what}: q, k and v must have the same number of tokens")
    ind, off = _i32(indptr), _i32(offsets)
    rows = min(ind.shape[0] - 1, off.shape[0])
    a = _lib.RopeArgs()
    a.q, a.q_stride_t, a.q_stride_h, a.num_qo_heads = q.data_ptr(), q.stride(0), q.stride(1), q.shape[1]
    a.k, a.k_stride_t, a.k_stride_h, a.num_kv_heads = k.data_ptr(), k.stride(0), k.stride(1), k.shape[1]
    if v is not None:
        a.v, a.v_stride_t, a.v_stride_h = v.data_ptr(), v.stride(0), v.stride(1)
    a.total_tokens, a.head_dim = T, 128
    keep = []
    if q_norm_weight is not None:
        qw = q_norm_weight.to(torch.bfloat16).contiguous()
        kw = k_norm_weight.to(torch.bfloat16).contiguous()
        keep += [qw, kw]
        a.q_norm_weight, a.k_norm_weight = qw.data_ptr(), kw.data_ptr()
        a.norm_eps, a.permute = float(eps), int(permute)
    a.rope_theta, a.rope_scale = float(config.rope_theta), float(config.rope_scale)
    if config.llama31:
        a.llama31 = 1
        a.low_freq_factor, a.high_freq_factor = float(config.low_freq_factor), float(config.high_freq_factor)
        a.old_context_len = float(config.original_max_position_embeddings)
    a.indptr, a.offsets, a.num_rows = ind.data_ptr(), off.data_ptr(), rows
    if kv_cache is not None:
        if kv_cache.dtype != torch.bfloat16 or kv_cache.stride(-1) != 1:
            raise ValueError(f"{what}: kv_cache must be bf16 with a contiguous head dim")
        pi, pp, lp = _i32(kv_page_indices), _i32(kv_page_indptr), _i32(kv_last_page_len)
        keep += [pi, pp, lp]
        a.kv_cache = kv_cache.data_ptr()
        a.cache_stride_p, a.cache_stride_kv, a.cache_stride_t, a.cache_stride_h = kv_cache.stride()[:4]
        a.page_size = int(page_size)
        a.kv_page_indices, a.kv_page_indptr, a.kv_last_page_len = pi.data_ptr(), pp.data_ptr(), lp.data_ptr()
        a.num_seq = lp.shape[0]
    a.write_k = int(write_k)
    _lib.check(_lib.lib().aspire_qk_norm_rope_append(ctypes.byref(a), _lib.stream_of(q)), what)


def apply_rope_inplace(q, k, indptr, offsets, config: RopeConfig | None = None) -> None:
    """``mylib::rope``: rotate q and k in place (interleaved pairs)."""
    _run(q, k, indptr, offsets, config=config or _CONFIG, what="mylib::rope")


def qk_norm_rope_update_kv(q, k, v, q_norm_weight, k_norm_weight, eps, kv_append_indptr, offsets, kv_cache,
                           kv_page_indices, kv_page_indptr, kv_last_page_len, page_size,
                           config: RopeConfig | None = None, permute: bool = True) -> None:
    """Norm (if weights are given), permute, rope and append k / v, in one launch; q in place."""
    _run(q, k, kv_append_indptr, offsets, config=config or _CONFIG, v=v, q_norm_weight=q_norm_weight,
         k_norm_weight=k_norm_weight, eps=eps, permute=permute, kv_cache=kv_cache, kv_page_indices=kv_page_indices,
         kv_page_indptr=kv_page_indptr, kv_last_page_len=kv_last_page_len, page_size=page_size,
         write_k=False, what="mylib::qk_norm_rope_update_kv")


_DEFINED = False


def define_rope_op(rope_base: float, scaling_factor: float = 1.0, low_freq_factor: float | None = None,
                   high_freq_factor: float | None = None, original_max_position_embeddings: int | None = None):
    """Register ``mylib::rope`` (and the fused op) for a model's rope settings, as setup_caches does."""
    global _DEFINED
    _CONFIG.rope_theta, _CONFIG.rope_scale = float(rope_base), float(scaling_factor)
    _CONFIG.low_freq_factor, _CONFIG.high_freq_factor = low_freq_factor, high_freq_factor
    _CONFIG.original_max_position_embeddings = original_max_position_embeddings
    if _DEFINED:
        return
    torch.library.define("mylib::rope", "(Tensor(a!) q, Tensor(b!) k, Tensor indptr, Tensor offsets) -> ()")
    torch.library.define(
        "mylib::qk_norm_rope_update_kv",
        "(Tensor(a!) q, Tensor k, Tensor v, Tensor? q_norm_weight, Tensor? k_norm_weight, float eps, "
        "Tensor kv_append_indptr, Tensor offsets, Tensor(b!) kv_cache, Tensor kv_page_indices, "
        "Tensor kv_page_indptr, Tensor kv_last_page_len, int page_size) -> ()")

    @torch.library.impl("mylib::rope", "cuda")
    def _rope(q, k, indptr, offsets):
        apply_rope_inplace(q, k, indptr, offsets)

    @torch.library.register_fake("mylib::rope")
    def _rope_fake(q, k, indptr, offsets):
        return None

    @torch.library.impl("mylib::qk_norm_rope_update_kv", "cuda")
    def _fused(q, k, v, q_norm_weight, k_norm_weight, eps, kv_append_indptr, offsets, kv_cache, kv_page_indices,
               kv_page_indptr, kv_last_page_len, page_size):
        qk_norm_rope_update_kv(q, k, v, q_norm_weight, k_norm_weight, eps, kv_append_indptr, offsets, kv_cache,
                               kv_page_indices, kv_page_indptr, kv_last_page_len, page_size)

    @torch.library.register_fake("mylib::qk_norm_rope_update_kv")
    def _fused_fake(*args):
        return None

    _DEFINED = True


__all__ = ["RopeConfig", "rope_frequencies", "apply_rope_inplace", "qk_norm_rope_update_kv", "define_rope_op"]
