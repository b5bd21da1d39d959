"""Mixed draft/verify paged attention wrapper (HIP implementation).

Drop-in for ``aspire/attention/holistic_wrapper.py``: ``HolisticAttentionWrapper``
keeps the reference constructor, ``plan`` / ``plan_host`` / ``run`` signatures
(holistic_wrapper.py:142-386) and ``build_holistic_dump_jit_args``
(holistic_wrapper.py:401-434).

* ``plan`` reads ``qo_indptr``, ``kv_indptr`` and the derived ``kv_len`` back to
  the host behind a stream synchronisation (holistic_wrapper.py:237-243) and
  then plans like ``plan_host``.
* ``plan_host`` runs the C++ planner of libaspire_hip.so on host arrays, writing
  a pinned staging slot and enqueuing its asynchronous upload to the device int
  workspace on the current stream. A ring of four event-fenced pinned slots
  makes reuse safe under host run-ahead (holistic_wrapper.py:180-198,316-342).
* ``run`` launches the persistent attention kernels (one per row-tile class)
  and the split-KV merge with fixed grids and fixed workspace pointers, so it
  can be captured in a HIP graph and replayed after later plans. With
  ``use_cuda_graph=True`` (or while the stream is capturing) every launch is
  issued; otherwise launches the current plan does not need are skipped.

The wrapper owns a 384 MiB float workspace (split-KV partial outputs), an
8 MiB int workspace (the plan) and 4 x 8 MiB of pinned staging, as the
reference does (holistic_wrapper.py:158-162).
"""

from __future__ import annotations

import ctypes
import math
from typing import List, Optional, Tuple, Union

import torch

from aspire_amd import _lib
from aspire_amd.backends.jit_kernels import (
    DumpVariant,
    _BASE_TENSOR_NAMES,
    _scalar_spec,
    _type_name,
    build_dump_struct,
)

FLOAT_WORKSPACE_BYTES = 384 * 1024 * 1024
INT_WORKSPACE_BYTES = 8 * 1024 * 1024
PINNED_RING = 4
# Plans of at most this many page-heads per wave are short launches whose end and merge wait on
# the split-KV partials: run() has them stored non-temporally (config 4 at f = 1.0, 32 per
# wave: 44.5 against 45.0 us on MI355X); longer plans keep plain stores.
SHORT_PLAN_PAGES_PER_WAVE = 64


def get_seq_lens(kv_indptr: torch.Tensor, kv_last_page_len: torch.Tensor, page_size: int) -> torch.Tensor:
    """``clamp(pages - 1, 0) * page_size + last_page_len`` per row (FlashInfer's get_seq_lens)."""
    n = kv_last_page_len.shape[0]
    pages = kv_indptr[1 : n + 1] - kv_indptr[:n]
    return (torch.clamp(pages - 1, min=0) * page_size + kv_last_page_len).to(torch.int32)


def _unpack_paged_kv_cache(paged_kv_cache, kv_layout: str):
    if kv_layout != "NHD":
        raise ValueError(f"only the NHD layout is supported, got {kv_layout!r}")
    if isinstance(paged_kv_cache, torch.Tensor):
        if paged_kv_cache.dim() != 5 or paged_kv_cache.shape[1] != 2:
            raise ValueError("paged_kv_cache must be [num_pages, 2, page_size, num_kv_heads, head_dim]")
        return paged_kv_cache[:, 0], paged_kv_cache[:, 1]
    if isinstance(paged_kv_cache, (tuple, list)) and len(paged_kv_cache) == 2:
        return paged_kv_cache[0], paged_kv_cache[1]
    raise ValueError("paged_kv_cache must be a tensor or a (k_cache, v_cache) pair")


class HolisticAttentionWrapper:
    """Drop-in replacement for the reference's holistic (persistent) attention wrapper."""

    def __init__(
        self,
        float_workspace_buffer: torch.Tensor,
        kv_layout: str = "NHD",
        use_cuda_graph: bool = False,
        qo_indptr_buf: Optional[torch.Tensor] = None,
        paged_kv_indptr_buf: Optional[torch.Tensor] = None,
        paged_kv_indices_buf: Optional[torch.Tensor] = None,
        paged_kv_last_page_len_buf: Optional[torch.Tensor] = None,
        jit_args: Optional[list] = None,
        jit_kwargs: Optional[dict] = None,
        *,
        waves_per_cu: Optional[int] = None,
        float_workspace_bytes: int = FLOAT_WORKSPACE_BYTES,
        **_ignored,
    ):
        if kv_layout != "NHD":
            raise ValueError(f"only the NHD layout is supported, got {kv_layout!r}")
        self._kv_layout = kv_layout
        self._use_cuda_graph = use_cuda_graph
        device = float_workspace_buffer.device
        _lib.require_cuda(float_workspace_buffer, what="HolisticAttentionWrapper")
        self._device = device
        self._float_workspace = torch.empty(float_workspace_bytes, dtype=torch.uint8, device=device)
        self._int_workspace = torch.empty(INT_WORKSPACE_BYTES, dtype=torch.uint8, device=device)
        self._pinned_ring = [
            torch.empty(INT_WORKSPACE_BYTES, dtype=torch.uint8, device="cpu", pin_memory=True)
            for _ in range(PINNED_RING)
        ]
        self._pinned_int_workspace = self._pinned_ring[0]
        self._pinned_ring_events: List[Optional[torch.cuda.Event]] = [None] * PINNED_RING
        self._pinned_slot = 0

        self._layout = _lib.PlanLayout()
        with torch.cuda.device(device):
            rc = _lib.lib().aspire_plan_layout_init(
                0, int(waves_per_cu or 0), INT_WORKSPACE_BYTES, float_workspace_bytes, 128,
                ctypes.byref(self._layout))
        _lib.check(rc, "HolisticAttentionWrapper")
        self._plan_info: Optional[_lib.PlanInfo] = None

        self._dump: Optional[DumpVariant] = None
        self._has_jit = jit_args is not None
        if jit_args is not None:
            spec = jit_args[12] if len(jit_args) > 12 else None
            if not isinstance(spec, DumpVariant):
                raise ValueError("jit_args must come from build_holistic_dump_jit_args / build_dump_jit_args")
            self._dump = spec

        self._kv_indices: Optional[torch.Tensor] = None
        self._page_size = 0
        self._sm_scale: Optional[float] = None
        self._causal = False
        self._num_qo_heads = 0
        self._num_kv_heads = 0
        self._planned = False

    # ------------------------------------------------------------------ plan
    def plan(
        self,
        qo_indptr: torch.Tensor,
        paged_kv_indptr: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        paged_kv_last_page_len: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim_qk: int,
        page_size: int,
        head_dim_vo: Optional[int] = None,
        q_data_type: Union[str, torch.dtype] = "float16",
        causal: bool = False,
        sm_scale: Optional[float] = None,
        **kwargs,
    ) -> None:
        kv_len = get_seq_lens(paged_kv_indptr, paged_kv_last_page_len, page_size)
        qo_host = qo_indptr.to("cpu", non_blocking=True)
        kv_indptr_host = paged_kv_indptr.to("cpu", non_blocking=True)
        kv_len_host = kv_len.to("cpu", non_blocking=True)
        torch.cuda.current_stream().synchronize()
        self._plan_from_host(qo_host, kv_indptr_host, kv_len_host, paged_kv_indices, num_qo_heads,
                             num_kv_heads, head_dim_qk, page_size, head_dim_vo, causal, sm_scale,
                             per_head_lists=False)

    def plan_host(
        self,
        qo_indptr_host: torch.Tensor,
        kv_indptr_host: torch.Tensor,
        kv_len_host: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim_qk: int,
        page_size: int,
        head_dim_vo: Optional[int] = None,
        causal: bool = False,
        sm_scale: Optional[float] = None,
        *,
        per_head_lists: bool = False,
    ) -> None:
        """Plan from host arrays with no device readback or synchronisation.

        The reference requires a prior ``plan()`` to resolve its JIT module
        (holistic_wrapper.py:302-306) and raises ``RuntimeError`` otherwise; the
        same contract is kept. ``per_head_lists`` (not in the reference) gives
        every (row, kv head) its own page list: ``kv_indptr_host`` then holds
        ``B*H_kv + 1`` entries and ``kv_len_host`` ``B*H_kv``.
        """
        if not self._planned:
            raise RuntimeError("plan_host requires a prior plan() call to resolve the kernel module")
        self._plan_from_host(qo_indptr_host, kv_indptr_host, kv_len_host, paged_kv_indices, num_qo_heads,
                             num_kv_heads, head_dim_qk, page_size, head_dim_vo, causal, sm_scale,
                             per_head_lists=per_head_lists)

    def plan_segments(
        self,
        qo_indptr_host: torch.Tensor,
        seg_start_host: torch.Tensor,
        seg_pages_host: torch.Tensor,
        seg_kv_len_host: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim_qk: int,
        page_size: int,
        head_dim_vo: Optional[int] = None,
        causal: bool = False,
        sm_scale: Optional[float] = None,
    ) -> None:
        """Plan per-(row, kv head) segments given by explicit list starts (not in the
        reference): segment ``b*H_kv + g`` streams ``seg_kv_len[s]`` tokens of the
        ``seg_pages[s]`` entries at ``paged_kv_indices[seg_start[s]]``. Rows whose
        heads share one start (verify rows over their block table) keep the
        row-list kernel path; rows with a list per head (the key-mean selection)
        read each head's own pages. Same preconditions as ``plan_host``."""
        if not self._planned:
            raise RuntimeError("plan_segments requires a prior plan() call to resolve the kernel module")
        self._plan_from_host(qo_indptr_host, None, seg_kv_len_host, paged_kv_indices, num_qo_heads, num_kv_heads,
                             head_dim_qk, page_size, head_dim_vo, causal, sm_scale, per_head_lists=True,
                             segments=(seg_start_host, seg_pages_host))

    def _plan_from_host(self, qo_host, kv_indptr_host, kv_len_host, paged_kv_indices, num_qo_heads,
                        num_kv_heads, head_dim_qk, page_size, head_dim_vo, causal, sm_scale, *,
                        per_head_lists: bool, segments=None) -> None:
        if head_dim_vo is None:
            head_dim_vo = head_dim_qk
        if head_dim_qk != 128 or head_dim_vo != 128:
            raise ValueError("the HIP attention kernel supports head_dim 128 only")
        qo = qo_host.to(torch.int32).contiguous()
        kvl = kv_len_host.to(torch.int32).contiguous()
        n_seg = kvl.shape[0]
        batch = n_seg // num_kv_heads if per_head_lists else n_seg
        if segments is not None:
            st = segments[0].to(torch.int32).contiguous()
            pg = segments[1].to(torch.int32).contiguous()
            if st.shape[0] < n_seg or pg.shape[0] < n_seg or n_seg % num_kv_heads:
                raise ValueError("segment arrays must hold batch * num_kv_heads entries")
            if n_seg and (int(st[:n_seg].min()) < 0 or int(pg[:n_seg].min()) < 0):
                raise ValueError("segment starts and page counts must be non-negative")
            if n_seg and int((st[:n_seg].long() + pg[:n_seg].long()).max()) > paged_kv_indices.numel():
                raise ValueError("paged_kv_indices is shorter than the segments describe")
            if qo.shape[0] < batch + 1:
                raise ValueError("plan arrays are shorter than the batch they describe")
        else:
            kvp = kv_indptr_host.to(torch.int32).contiguous()
            if qo.shape[0] < batch + 1 or kvp.shape[0] < n_seg + 1:
                raise ValueError("plan arrays are shorter than the batch they describe")
            if n_seg and int(kvp[: n_seg + 1].max()) > paged_kv_indices.numel():
                raise ValueError("paged_kv_indices is shorter than kv_indptr describes")
        if int(qo[: batch + 1].min()) < 0:
            raise ValueError("qo_indptr must be non-negative")
        slot = self._pinned_slot
        event = self._pinned_ring_events[slot]
        if event is not None:
            event.synchronize()
        info = _lib.PlanInfo()
        buf = self._pinned_ring[slot]
        if segments is not None:
            rc = _lib.lib().aspire_plan_build_segments(
                ctypes.byref(self._layout), _lib.ptr(qo), _lib.ptr(st), _lib.ptr(pg), _lib.ptr(kvl), batch,
                num_qo_heads, num_kv_heads, page_size, 1 if causal else 0, _lib.ptr(buf), buf.numel(),
                ctypes.byref(info))
        else:
            rc = _lib.lib().aspire_plan_build(
                ctypes.byref(self._layout), _lib.ptr(qo), _lib.ptr(kvp), _lib.ptr(kvl), batch,
                1 if per_head_lists else 0, num_qo_heads, num_kv_heads, page_size, 1 if causal else 0,
                _lib.ptr(buf), buf.numel(), ctypes.byref(info))
        _lib.check(rc, "plan")
        stream = torch.cuda.current_stream(self._device)
        rc = _lib.lib().aspire_plan_upload(ctypes.byref(self._layout), ctypes.byref(info), _lib.ptr(buf),
                                           _lib.ptr(self._int_workspace), ctypes.c_void_p(stream.cuda_stream))
        _lib.check(rc, "plan")
        if event is None:
            event = torch.cuda.Event()
            self._pinned_ring_events[slot] = event
        event.record(stream)
        self._pinned_slot = (slot + 1) % PINNED_RING

        self._plan_info = info
        self._plan_tokens = int(qo[: batch + 1].max()) if batch else 0
        # rows that can write dump entries / page scores: queries and at least one page
        if per_head_lists:
            has_kv = (kvl[: batch * num_kv_heads].view(batch, num_kv_heads) > 0).any(dim=1) if batch else kvl[:0]
        else:
            has_kv = kvl[:batch] > 0
        writes = ((qo[1 : batch + 1] - qo[:batch]) > 0) & has_kv
        nz = torch.nonzero(writes)
        self._plan_batch = int(nz.max()) + 1 if nz.numel() else 0
        self._plan_max_kv = int(kvl.max()) if n_seg else 0
        self._plan_max_pages = (self._plan_max_kv + page_size - 1) // page_size
        self._kv_indices = paged_kv_indices
        self._page_size = page_size
        self._sm_scale = sm_scale
        self._causal = bool(causal)
        self._num_qo_heads = num_qo_heads
        self._num_kv_heads = num_kv_heads
        self._planned = True

    @property
    def plan_info(self) -> Optional[_lib.PlanInfo]:
        return self._plan_info

    # ------------------------------------------------------------------- run
    def run(
        self,
        q: torch.Tensor,
        paged_kv_cache: Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]],
        *args,
        out: Optional[torch.Tensor] = None,
        return_lse: bool = False,
        page_scores: Optional[torch.Tensor] = None,
        **kwargs,
    ):
        """``run(q, kv_cache[, dump_buffer, [mode_flags], num_heads, jit_kv_stride], out=, return_lse=)``.

        ``page_scores`` (not in the reference) receives the per-KV-head key-mean
        page scores ``[B*H_kv, max_pages]`` fp32 of single-query rows.
        """
        if not self._planned:
            raise RuntimeError("run() requires plan() or plan_host() first")
        k_cache, v_cache = _unpack_paged_kv_cache(paged_kv_cache, self._kv_layout)
        _lib.require_cuda(q, k_cache, v_cache, what="HolisticAttentionWrapper.run")
        if q.dim() != 3 or q.shape[2] != 128 or q.stride(2) != 1:
            raise ValueError("q must be [T, num_qo_heads, 128] with a contiguous head dimension")
        if q.shape[1] != self._num_qo_heads:
            raise ValueError(f"q has {q.shape[1]} heads, plan has {self._num_qo_heads}")
        if q.dtype != torch.bfloat16 or k_cache.dtype != torch.bfloat16:
            raise ValueError("the HIP attention kernel computes in bf16 (q and kv_cache)")
        if k_cache.stride() != v_cache.stride() or k_cache.stride(3) != 1:
            raise ValueError("k and v caches must share strides with a contiguous head dimension")
        if k_cache.shape[1] != self._page_size or k_cache.shape[2] != self._num_kv_heads:
            raise ValueError("kv_cache page size / kv heads disagree with the plan")
        if q.shape[0] < self._plan_tokens:
            raise ValueError(f"q has {q.shape[0]} tokens, the plan addresses {self._plan_tokens}")
        if out is None:
            out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        if out.shape != q.shape or out.stride(2) != 1 or out.dtype != q.dtype:
            raise ValueError("out must match q's shape and dtype with a contiguous head dimension")
        lse = torch.empty(q.shape[0], q.shape[1], device=q.device, dtype=torch.float32)
        sm_scale = self._sm_scale if self._sm_scale is not None else 1.0 / math.sqrt(q.shape[2])
        elem = k_cache.element_size()
        kv_off = (v_cache.data_ptr() - k_cache.data_ptr())
        if kv_off % elem:
            raise ValueError("v_cache is not element-aligned with k_cache")

        a = _lib.AttentionArgs()
        a.q, a.q_stride_t, a.q_stride_h = q.data_ptr(), q.stride(0), q.stride(1)
        a.kv_cache = k_cache.data_ptr()
        a.cache_stride_p, a.cache_stride_kv = k_cache.stride(0), kv_off // elem
        a.cache_stride_t, a.cache_stride_h = k_cache.stride(1), k_cache.stride(2)
        a.kv_indices = self._kv_indices.data_ptr()
        a.out, a.out_stride_t, a.out_stride_h = out.data_ptr(), out.stride(0), out.stride(1)
        a.lse = lse.data_ptr()
        a.plan_dev = self._int_workspace.data_ptr()
        a.float_ws = self._float_workspace.data_ptr()
        a.num_qo_heads, a.num_kv_heads = self._num_qo_heads, self._num_kv_heads
        a.head_dim, a.page_size = 128, self._page_size
        a.sm_scale, a.causal = float(sm_scale), 1 if self._causal else 0
        info = self._plan_info
        if self._use_cuda_graph or torch.cuda.is_current_stream_capturing():
            a.class_mask, a.launch_merge = 7, 1
        else:
            a.class_mask = sum(1 << c for c in range(3) if info.num_items[c] > 0)
            a.launch_merge = 1 if info.num_merge > 0 else 0
        # short plans store their split-KV partials non-temporally (a graph keeps the choice
        # of the plan it was captured with; either is correct for any plan)
        a.partial_nt = 1 if info.total_pages <= SHORT_PLAN_PAGES_PER_WAVE * self._layout.num_waves else 0
        keep_alive = [q, out, lse]
        wants_dump = self._has_jit and self._dump is not None and self._dump.kind != "noop"
        if (wants_dump or page_scores is not None) and info.split_rows > 0:
            raise ValueError("the logits dump and page scores need whole rows; this plan cut rows longer "
                             "than 48 query rows into query tiles")
        if wants_dump:
            dump_buffer = args[0]
            rest = list(args[1:])
            mode_flags = rest.pop(0) if self._dump.use_mode_flags else None
            num_heads, kv_stride = int(rest[0]), int(rest[1])
            if dump_buffer.dtype not in (torch.float16, torch.float32):
                raise ValueError("dump buffer must be fp16 or fp32")
            if num_heads < self._num_qo_heads or kv_stride < self._plan_max_kv:
                raise ValueError("dump num_heads / kv_stride smaller than the planned heads / kv lengths")
            if dump_buffer.numel() < self._plan_batch * num_heads * self._dump.slots * kv_stride:
                raise ValueError("dump buffer smaller than batch * num_heads * slots * kv_stride")
            if not dump_buffer.is_contiguous():
                raise ValueError("dump buffer must be contiguous")
            _lib.require_cuda(dump_buffer, what="HolisticAttentionWrapper.run")
            a.dump = dump_buffer.data_ptr()
            a.dump_kind = self._dump.kernel_kind
            a.dump_dtype = 1 if dump_buffer.dtype == torch.float32 else 0
            a.dump_kv_stride, a.dump_num_heads = kv_stride, num_heads
            if mode_flags is not None:
                mf = mode_flags.to(torch.int32).contiguous()
                keep_alive.append(mf)
                a.dump_mode_flags = mf.data_ptr()
        if page_scores is not None:
            if page_scores.dtype != torch.float32 or page_scores.stride(-1) != 1 or page_scores.dim() != 2:
                raise ValueError("page_scores must be a 2-D fp32 tensor with a contiguous last dimension")
            if (page_scores.shape[0] < self._plan_batch * self._num_kv_heads
                    or page_scores.shape[1] < self._plan_max_pages):
                raise ValueError("page_scores must be at least [batch * num_kv_heads, max pages]")
            a.page_scores = page_scores.data_ptr()
            a.page_score_stride = page_scores.stride(0)
        rc = _lib.lib().aspire_attention_run(ctypes.byref(self._layout), ctypes.byref(a), _lib.stream_of(q))
        _lib.check(rc, "HolisticAttentionWrapper.run")
        if return_lse:
            return out, lse
        return out


def build_holistic_dump_jit_args(
    dtype: torch.dtype,
    head_dim: int,
    dump_kind: str = "last_token",
    class_name: str = "HolisticDumpAttentionWeights",
    op_name: str = "holistic_batch_dump_attention_weights",
    use_mode_flags: bool = False,
    dump_buffer_dtype: torch.dtype = torch.float32,
) -> list:
    """Dump-variant arguments in the reference's list shape (holistic_wrapper.py:401-434).

    ``wrapper.run(q, kv_cache, attention_weights_buf, [mode_flags], num_heads,
    jit_kv_stride, return_lse=..., out=...)``.
    """
    scalar_names, scalar_types = _scalar_spec("holistic")
    attn_type = _type_name(dump_buffer_dtype)
    spec = build_dump_struct("holistic", dump_kind, class_name, use_mode_flags, attn_type=attn_type)
    tensor_names = list(_BASE_TENSOR_NAMES)
    tensor_types = [attn_type]
    if use_mode_flags and dump_kind != "noop":
        tensor_names.append("mode_flags")
        tensor_types.append("int32_t")
    return [op_name, dtype, dtype, dtype, torch.int32, head_dim, head_dim, tensor_names, tensor_types,
            scalar_names, scalar_types, class_name, spec]


def define_unified_decode_op(wrapper: HolisticAttentionWrapper, op_name: str = "mylib::unified_decode"):
    """Register ``mylib::unified_decode(Tensor q, Tensor kv_cache, Tensor(a!) out) -> ()`` over
    ``wrapper`` (aspire/models/sparse_draft_runner.py:599-612): the op runs the planned mixed
    attention into ``out``; its fake implementation returns nothing, so torch.compile traces
    the call without running it."""
    torch.library.define(op_name, "(Tensor q, Tensor kv_cache, Tensor(a!) out) -> ()")

    @torch.library.impl(op_name, "cuda")
    def _unified_decode(q, kv_cache, out):
        wrapper.run(q, kv_cache, out=out)

    @torch.library.register_fake(op_name)
    def _unified_decode_fake(q, kv_cache, out):
        return None

    return getattr(torch.ops.mylib, op_name.split("::", 1)[1])


def define_dump_op(wrapper: HolisticAttentionWrapper, op_name: str, num_heads: int, kv_stride: int,
                   mode_flags: Optional[torch.Tensor] = None):
    """Register the refresh layer's dump op ``(Tensor q, Tensor kv_cache, Tensor(a!) dump_buffer,
    Tensor(b!) out) -> Tensor`` over a wrapper built with dump ``jit_args``
    (aspire/backends/base.py:452-489): it runs the full attention, writes the logits dump and
    returns the base-2 LSE ``[T, num_heads]`` fp32 (its fake implementation returns an empty one)."""
    torch.library.define(op_name, "(Tensor q, Tensor kv_cache, Tensor(a!) dump_buffer, Tensor(b!) out) -> Tensor")

    @torch.library.impl(op_name, "cuda")
    def _dump_kernel(q, kv_cache, dump_buffer, out):
        args = [q, kv_cache, dump_buffer] + ([mode_flags] if mode_flags is not None else []) + [num_heads, kv_stride]
        _, lse = wrapper.run(*args, return_lse=True, out=out)
        return lse

    @torch.library.register_fake(op_name)
    def _dump_kernel_fake(q, kv_cache, dump_buffer, out):
        return torch.empty((q.shape[0], num_heads), dtype=torch.float32, device=q.device)

    return getattr(torch.ops.mylib, op_name.split("::", 1)[1])
