"""Chunked-prefill paged attention: drop-in for ``flashinfer.BatchPrefillWithPagedKVCacheWrapper``.

The reference plans and runs FlashInfer's paged prefill wrapper for prompt chunks
(aspire/models/sparse_draft_runner.py:199-209; the chunk loop of ``encode_slots``,
aspire/backends/base.py:1559-1674): causal attention of each row's new tokens over its
cached prefix plus the new tokens, page lists as for decode. ``run`` launches the
dedicated prefill kernel (``aspire_prefill_run``): each workgroup takes one query block
(``aspire_prefill_block_tokens(hq, hkv)`` tokens of one row, all G query heads of one kv
head) and stages every page of its keys once in LDS, two pages per step, for all of its
waves (head groups that do not divide a wave's 32 query rows take the decode path below).
``kernel="decode"`` runs the mixed decode kernel and its
planner instead (rows cut into 48-query-row tiles). ``plan`` / ``run`` keep FlashInfer's
names and argument meanings; options this path does not implement (custom masks, sliding
windows, logit soft caps, fused RoPE) raise ``ValueError``.

Graph replay: the reference builds its decode and draft wrappers of this class with
``use_cuda_graph=True`` and replays their captured ``run`` after every re-plan
(sparse_draft_runner.py:261-268,297-303). The prefill kernel's launch bakes in the plan's
block count and per-plan index tensors, so with ``use_cuda_graph=True``, or whenever ``run``
is called while the stream is capturing, the wrapper runs the decode kernel's plan instead:
its launches read the plan from the wrapper's fixed int workspace (fixed grid, fixed
pointers), so a graph captured after one plan replays any later one correctly.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Union

import torch

from aspire_amd import _lib
from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper, _unpack_paged_kv_cache


class BatchPrefillWithPagedKVCacheWrapper(HolisticAttentionWrapper):
    def __init__(self, float_workspace_buffer: torch.Tensor, kv_layout: str = "NHD", use_cuda_graph: bool = False,
                 qo_indptr_buf: Optional[torch.Tensor] = None, paged_kv_indptr_buf: Optional[torch.Tensor] = None,
                 paged_kv_indices_buf: Optional[torch.Tensor] = None,
                 paged_kv_last_page_len_buf: Optional[torch.Tensor] = None, backend: str = "auto",
                 jit_args: Optional[list] = None, jit_kwargs: Optional[dict] = None, *, kernel: str = "prefill",
                 **kwargs):
        if kernel not in ("prefill", "decode"):
            raise ValueError("kernel must be 'prefill' or 'decode'")
        self._kernel = kernel
        self._pf = None
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
        self._pf = None
        if self._kernel != "prefill" or self._has_jit or self._use_cuda_graph:
            # graph-mode wrappers keep the decode kernel's fixed-pointer plan (module docstring)
            return
        bt = int(_lib.lib().aspire_prefill_block_tokens(num_qo_heads, num_kv_heads))
        if bt <= 0:
            # a head group that does not divide a wave's 32 query rows (e.g. 6 or 12 query heads
            # per kv head): the mixed kernel's query tiles serve the plan made above
            return
        # rows: the entries of kv_last_page_len (FlashInfer's batch), with their query blocks
        n = paged_kv_last_page_len.shape[0]
        qo_host = qo_indptr[: n + 1].to("cpu", torch.int64)
        q_len = (qo_host[1:] - qo_host[:-1]).clamp(min=0)
        blocks = torch.zeros(n + 1, dtype=torch.int64)
        blocks[1:] = torch.cumsum((q_len + bt - 1) // bt, 0)
        dev = paged_kv_indices.device
        self._pf = {
            "qo": qo_indptr[: n + 1].to(dev, torch.int32).contiguous(),
            "kvp": paged_kv_indptr[: n + 1].to(dev, torch.int32).contiguous(),
            "lpl": paged_kv_last_page_len[:n].to(dev, torch.int32).contiguous(),
            "idx": paged_kv_indices.to(torch.int32).contiguous(),
            "blocks": blocks.to(dev, torch.int32),
            "rows": n, "total_blocks": int(blocks[-1]), "block_tokens": bt,
            "tokens": int(qo_host[-1]) if n else 0,
        }

    def run(self, q: torch.Tensor, paged_kv_cache, *args, out: Optional[torch.Tensor] = None,
            lse: Optional[torch.Tensor] = None, return_lse: bool = False, **kwargs):
        if self._pf is None or torch.cuda.is_current_stream_capturing():
            # the decode kernel's plan: also the path a capture records, since its launches
            # read the plan from the fixed int workspace and stay valid after later plans
            res = super().run(q, paged_kv_cache, *args, out=out, return_lse=True)
            o, l_ = res
            if lse is not None:
                lse.copy_(l_)
                l_ = lse
            return (o, l_) if return_lse else o
        pf = self._pf
        k_cache, v_cache = _unpack_paged_kv_cache(paged_kv_cache, self._kv_layout)
        _lib.require_cuda(q, k_cache, v_cache, what="BatchPrefillWithPagedKVCacheWrapper.run")
        if q.dim() != 3 or q.shape[2] != 128 or q.stride(2) != 1 or q.dtype != torch.bfloat16:
            raise ValueError("q must be bf16 [T, num_qo_heads, 128] with a contiguous head dimension")
        if q.shape[1] != self._num_qo_heads or q.shape[0] < pf["tokens"]:
            raise ValueError("q's heads / tokens disagree with the plan")
        if k_cache.dtype != torch.bfloat16 or k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
            raise ValueError("kv_cache must be bf16 with k and v sharing strides and a contiguous head dimension")
        if k_cache.shape[1] != self._page_size or k_cache.shape[2] != self._num_kv_heads:
            raise ValueError("kv_cache page size / kv heads disagree with the plan")
        if out is None:
            out = torch.empty_like(q)
        if out.shape != q.shape or out.stride(2) != 1 or out.dtype != q.dtype:
            raise ValueError("out must match q's shape and dtype with a contiguous head dimension")
        want_lse = return_lse or lse is not None
        if lse is None and want_lse:
            lse = torch.empty(q.shape[0], q.shape[1], device=q.device, dtype=torch.float32)
        if lse is not None and (lse.dtype != torch.float32 or not lse.is_contiguous()
                                or tuple(lse.shape) != (q.shape[0], q.shape[1])):
            raise ValueError("lse must be a contiguous fp32 [T, num_qo_heads] tensor")
        elem = k_cache.element_size()
        a = _lib.PrefillArgs()
        a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
        a.kv_cache = k_cache.data_ptr()
        a.cache_stride_p, a.cache_stride_kv = k_cache.stride(0), (v_cache.data_ptr() - k_cache.data_ptr()) // elem
        a.cache_stride_t, a.cache_stride_h = k_cache.stride(1), k_cache.stride(2)
        a.kv_indices, a.kv_indptr = pf["idx"].data_ptr(), pf["kvp"].data_ptr()
        a.kv_last_page_len, a.qo_indptr, a.block_indptr = pf["lpl"].data_ptr(), pf["qo"].data_ptr(), pf["blocks"].data_ptr()
        a.num_rows, a.total_blocks, a.block_tokens = pf["rows"], pf["total_blocks"], pf["block_tokens"]
        a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
        a.lse = lse.data_ptr() if lse is not None else None
        a.num_qo_heads, a.num_kv_heads, a.head_dim, a.page_size = self._num_qo_heads, self._num_kv_heads, 128, 16
        a.sm_scale = float(self._sm_scale if self._sm_scale is not None else 1.0 / math.sqrt(128))
        a.causal = 1 if self._causal else 0
        rc = _lib.lib().aspire_prefill_run(ctypes.byref(a), _lib.stream_of(q))
        _lib.check(rc, "BatchPrefillWithPagedKVCacheWrapper.run")
        return (out, lse) if return_lse else out

    forward = run


__all__ = ["BatchPrefillWithPagedKVCacheWrapper"]
