"""Chunked-prefill paged attention: drop-in for ``flashinfer.BatchPrefillWithPagedKVCacheWrapper``.

The reference plans and runs FlashInfer's paged prefill wrapper for prompt chunks
(aspire/models/sparse_draft_runner.py:199-209; the chunk loop of ``encode_slots``,
aspire/backends/base.py:1559-1674): causal attention of each row's new tokens over its
cached prefix plus the new tokens, page lists as for decode. Here it is the same HIP
kernel and planner as the mixed decode path: rows longer than one 48-query-row item are
cut by the planner into query tiles whose keys end at the tile's last token. ``plan`` /
``run`` keep FlashInfer's names and argument meanings; options this path does not
implement (custom masks, sliding windows, logit soft caps, fused RoPE) raise
``ValueError``.
"""

from __future__ import annotations

from typing import Optional, Union

import torch

from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper


class BatchPrefillWithPagedKVCacheWrapper(HolisticAttentionWrapper):
    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD", use_cuda_graph: bool = False,
                 qo_indptr_buf: Optional[torch.Tensor] = None, paged_kv_indptr_buf: Optional[torch.Tensor] = None,
                 paged_kv_indices_buf: Optional[torch.Tensor] = None,
                 paged_kv_last_page_len_buf: Optional[torch.Tensor] = None, backend: str = "auto",
                 jit_args: Optional[list] = None, jit_kwargs: Optional[dict] = None, **kwargs):
        super().__init__(float_workspace_buffer, kv_layout, use_cuda_graph=use_cuda_graph,
                         qo_indptr_buf=qo_indptr_buf, paged_kv_indptr_buf=paged_kv_indptr_buf,
                         paged_kv_indices_buf=paged_kv_indices_buf,
                         paged_kv_last_page_len_buf=paged_kv_last_page_len_buf, jit_args=jit_args,
                         jit_kwargs=jit_kwargs, **kwargs)

    def plan(self, qo_indptr: torch.Tensor, paged_kv_indptr: torch.Tensor, paged_kv_indices: torch.Tensor,
             paged_kv_last_page_len: torch.Tensor, num_qo_heads: int, num_kv_heads: int, head_dim_qk: int,
             page_size: int, head_dim_vo: Optional[int] = None, custom_mask: Optional[torch.Tensor] = None,
             packed_custom_mask: Optional[torch.Tensor] = None, causal: bool = False,
             pos_encoding_mode: str = "NONE", use_fp16_qk_reduction: bool = False, sm_scale: Optional[float] = None,
             window_left: int = -1, logits_soft_cap: Optional[float] = None, rope_scale: Optional[float] = None,
             rope_theta: Optional[float] = None, q_data_type: Union[str, torch.dtype] = "float16",
             kv_data_type=None, non_blocking: bool = True, **kwargs) -> None:
        if custom_mask is not None or packed_custom_mask is not None:
            raise ValueError("custom masks are not supported by the HIP prefill path")
        if pos_encoding_mode != "NONE" or rope_scale is not None or rope_theta is not None:
            raise ValueError("fused RoPE is not supported here; apply mylib::rope before run()")
        if window_left != -1 or logits_soft_cap not in (None, 0.0):
            raise ValueError("sliding windows and logit soft caps are not supported by the HIP prefill path")
        super().plan(qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, num_qo_heads,
                     num_kv_heads, head_dim_qk, page_size, head_dim_vo=head_dim_vo, q_data_type=q_data_type,
                     causal=causal, sm_scale=sm_scale)

    def run(self, q: torch.Tensor, paged_kv_cache, *args, out: Optional[torch.Tensor] = None,
            lse: Optional[torch.Tensor] = None, return_lse: bool = False, **kwargs):
        res = super().run(q, paged_kv_cache, *args, out=out, return_lse=True)
        o, l_ = res
        if lse is not None:
            lse.copy_(l_)
            l_ = lse
        return (o, l_) if return_lse else o

    forward = run


__all__ = ["BatchPrefillWithPagedKVCacheWrapper"]
