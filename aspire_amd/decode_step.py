"""One full mixed draft/verify decode step of a Qwen3-shape model on the HIP path.

The step follows ``TransformerSparseDraft.unified_forward``
(aspire/models/sparse_draft_transformer.py:242-286) and its layers
(``TransformerBlockSparseDraft.unified_forward``, :224-239;
``AttentionSparseDraft.unified_forward``, :140-177):

    x = tok_embeddings(ids)
    per layer: a = attention_norm(x); q, k, v = wqkv(a); q/k RMSNorm + rotary permute
               + RoPE + KV append; y = attention(q); x += wo(y)
               f = ffn_norm(x); x += w2(silu(w1 f) * w3 f)
    logits = output(norm(x)); ids = argmax(logits)

The GEMMs are torch's (hipBLASLt). The q/k preparation and the append are one
launch (``qk_norm_rope_update_kv``), the attention is ``HolisticAttentionWrapper``,
and the residual adds, norms, SwiGLU step and token pick are the row kernels of
the HIP library (``aspire_add_rms_norm``, ``aspire_silu_mul``,
``aspire_argmax_rows``), so a whole step can be recorded in one HIP graph.

Refresh layer, ``selector="keymean"`` (BASELINE config 2's selection): at
``refresh_layer`` every row attends its full context and the kernel writes the
key-mean page scores of the single-query (draft) rows; the top-``budget`` pages
per (row, KV head), the last ``recent_pages`` forced in, become the draft rows'
per-head page lists (verify rows keep one shared list, their full table, and the
kernel's staged row path) for the layers after it, and for the layers before it
in the next step. Before the first step every draft segment lists its row's last
``budget`` pages.

Refresh layer, ``selector="first_last"`` (the reference's own selection): the
refresh layer's full attention also writes the fp16 first/last logits dump of
every row and its LSE (the dump op of base.py:452-514); at the start of the next
step, as the reference's step preparation does (base.py:580-667,708-716),
``PageSelectorFirstLastAvg`` selects each row's top-``budget`` pages from them
(the last ``recent_pages`` forced in, default 8 as config.py:29), and
``build_unified_indices`` makes one page list per row (the draft rows' selection,
the verify rows' table; base.py:1200-1256) that every layer of the step except
the refresh layer attends, on the kernel's staged row path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F

from aspire_amd import _lib
from aspire_amd.attention.holistic_wrapper import HolisticAttentionWrapper, build_holistic_dump_jit_args
from aspire_amd.attention.page_list import build_head_page_lists, build_unified_indices
from aspire_amd.attention.rope import RopeConfig, qk_norm_rope_update_kv
from aspire_amd.backends.page_selector import KeyMeanPageSelector, PageSelectorFirstLastAvg

PAGE = 16
DRAFT_MODE, VERIFY_MODE = 0, 1


@dataclass(frozen=True)
class ModelShape:
    """The ``ModelArgs`` fields a decode step needs (aspire/models/transformer.py:22-49)."""

    n_layer: int = 36
    dim: int = 4096
    n_head: int = 32
    n_local_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 12288
    vocab_size: int = 151936
    rope_base: float = 1e6
    norm_eps: float = 1e-6
    use_qk_norm: bool = True

    @property
    def q_size(self) -> int:
        return self.n_head * self.head_dim

    @property
    def kv_size(self) -> int:
        return self.n_local_heads * self.head_dim

    @property
    def layer_params(self) -> int:
        d, i = self.dim, self.intermediate_size
        return (self.q_size + 2 * self.kv_size) * d + self.q_size * d + 2 * i * d + i * d + 2 * d + 2 * self.head_dim


# "Qwen3-8b" of transformer.py:90
QWEN3_8B = ModelShape()


# ------------------------------------------------------------------ row ops
def _bf16_rows(t: torch.Tensor, name: str) -> None:
    if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D bf16 tensor with contiguous rows")


def add_rms_norm(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor, eps: float,
                 delta: torch.Tensor | None = None) -> torch.Tensor:
    """``x += delta`` (when given), then ``out = RMSNorm(x) * weight`` (bf16, row-wise)."""
    _lib.require_cuda(x, weight, out, what="add_rms_norm")
    _bf16_rows(x, "x")
    _bf16_rows(out, "out")
    if delta is not None:
        _bf16_rows(delta, "delta")
        if delta.shape != x.shape:
            raise ValueError("add_rms_norm: delta must match x")
    if weight.dtype != torch.bfloat16 or not weight.is_contiguous() or weight.numel() != x.shape[1]:
        raise ValueError("add_rms_norm: weight must be a contiguous bf16 vector of x's width")
    if out.shape != x.shape:
        raise ValueError("add_rms_norm: out must match x")
    rc = _lib.lib().aspire_add_rms_norm(
        _lib.ptr(x), x.stride(0), _lib.ptr(delta), delta.stride(0) if delta is not None else 0, _lib.ptr(weight),
        _lib.ptr(out), out.stride(0), x.shape[0], x.shape[1], float(eps), _lib.stream_of(x))
    _lib.check(rc, "add_rms_norm")
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """``out = silu(gate_up[:, :I]) * gate_up[:, I:]`` with the reference's two bf16 roundings."""
    _lib.require_cuda(gate_up, out, what="silu_mul")
    _bf16_rows(gate_up, "gate_up")
    _bf16_rows(out, "out")
    inter = out.shape[1]
    if gate_up.shape != (out.shape[0], 2 * inter):
        raise ValueError("silu_mul: gate_up must be [T, 2 * I] for out [T, I]")
    rc = _lib.lib().aspire_silu_mul(_lib.ptr(gate_up), gate_up.stride(0), _lib.ptr(out), out.stride(0),
                                    out.shape[0], inter, _lib.stream_of(out))
    _lib.check(rc, "silu_mul")
    return out


def argmax_rows(logits: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """``ids[r] = argmax(logits[r])`` (first index of the maximum)."""
    _lib.require_cuda(logits, ids, what="argmax_rows")
    _bf16_rows(logits, "logits")
    if ids.dtype != torch.int64 or not ids.is_contiguous() or ids.numel() < logits.shape[0]:
        raise ValueError("argmax_rows: ids must be a contiguous int64 tensor with one entry per row")
    rc = _lib.lib().aspire_argmax_rows(_lib.ptr(logits), logits.stride(0), logits.shape[0], logits.shape[1],
                                       _lib.ptr(ids), _lib.stream_of(logits))
    _lib.check(rc, "argmax_rows")
    return ids


# ------------------------------------------------------------------ weights
def _fill_normal(t: torch.Tensor, gen: torch.Generator, std: float, mean: float = 0.0) -> torch.Tensor:
    return t.normal_(mean, std, generator=gen)


class DecodeWeights:
    """Random-init bf16 weights in the reference's module layout, with ``wqkv`` as
    ``[q | k | v]`` rows (transformer.py's fused projection) and ``w13`` as the
    ``w1`` (gate) rows followed by the ``w3`` (up) rows. Linear weights are
    N(0, 1/fan_in); norm weights N(1, 0.1^2); embeddings N(0, 1)."""

    def __init__(self, shape: ModelShape, device, seed: int = 0):
        self.shape = shape
        dev = torch.device(device)
        gen = torch.Generator(device=dev).manual_seed(seed)
        d, i = shape.dim, shape.intermediate_size
        bf = torch.bfloat16

        def lin(out_f, in_f):
            return _fill_normal(torch.empty(out_f, in_f, dtype=bf, device=dev), gen, 1.0 / math.sqrt(in_f))

        def norm(n):
            return _fill_normal(torch.empty(n, dtype=bf, device=dev), gen, 0.1, 1.0)

        self.tok_embeddings = _fill_normal(torch.empty(shape.vocab_size, d, dtype=bf, device=dev), gen, 1.0)
        self.layers = []
        for _ in range(shape.n_layer):
            self.layers.append(dict(
                attention_norm=norm(d),
                wqkv=lin(shape.q_size + 2 * shape.kv_size, d),
                q_norm=norm(shape.head_dim) if shape.use_qk_norm else None,
                k_norm=norm(shape.head_dim) if shape.use_qk_norm else None,
                wo=lin(d, shape.q_size),
                ffn_norm=norm(d),
                w13=lin(2 * i, d),
                w2=lin(d, i),
            ))
        self.norm = norm(d)
        self.output = lin(shape.vocab_size, d)

    def layer_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.layers[0].values() if t is not None)

    def to(self, device) -> "DecodeWeights":
        """A copy on ``device`` (test helper: the CPU restatement runs on host copies)."""
        new = object.__new__(DecodeWeights)
        new.shape = self.shape
        new.tok_embeddings = self.tok_embeddings.to(device)
        new.layers = [{k: (v.to(device) if v is not None else None) for k, v in l.items()} for l in self.layers]
        new.norm = self.norm.to(device)
        new.output = self.output.to(device)
        return new


def alloc_kv_caches(shape: ModelShape, pool_pages: int, device, seed: int = 0) -> torch.Tensor:
    """``[n_layer, pool_pages, 2, 16, H_kv, 128]`` bf16 page pools filled with N(0, 1)."""
    caches = torch.empty(shape.n_layer, pool_pages, 2, PAGE, shape.n_local_heads, shape.head_dim,
                         dtype=torch.bfloat16, device=device)
    gen = torch.Generator(device=caches.device).manual_seed(seed + 5)
    for layer in range(shape.n_layer):
        _fill_normal(caches[layer], gen, 1.0)
    return caches


# --------------------------------------------------------------------- step
class MixedDecodeStep:
    """The decode step's buffers, plans and forward for one batch of rows.

    ``ctx_len`` is each row's KV length after this step's append (its new tokens
    are the last ``q_len`` positions); ``is_draft`` rows have ``q_len`` 1.
    ``block_table`` is ``[B, W]`` int32 (logical -> physical page) into
    ``caches`` (``alloc_kv_caches``), shared by every layer.
    """

    def __init__(self, weights: DecodeWeights, caches: torch.Tensor, ctx_len, q_len, is_draft,
                 block_table: torch.Tensor, *, budget: int = 128, refresh_layer: int = 2,
                 recent_pages: int | None = None, selector: str = "keymean", tokens: torch.Tensor | None = None,
                 seed: int = 0, waves_per_cu: int | None = None):
        if selector not in ("keymean", "first_last"):
            raise ValueError("selector must be 'keymean' or 'first_last'")
        self.selector_kind = selector
        if recent_pages is None:
            recent_pages = 8 if selector == "first_last" else 1
        shape = weights.shape
        self.shape, self.w, self.caches = shape, weights, caches
        dev = caches.device
        self.device = dev
        ctx = np.asarray(ctx_len, dtype=np.int64)
        ql = np.asarray(q_len, dtype=np.int64)
        dr = np.asarray(is_draft, dtype=bool)
        if np.any(ql[dr] != 1):
            raise ValueError("draft rows have q_len 1")
        if np.any(ctx < ql) or np.any(ql < 1):
            raise ValueError("every row needs q_len >= 1 new tokens inside its context")
        if shape.head_dim != 128 or shape.n_head % shape.n_local_heads:
            raise ValueError("head_dim 128 and whole GQA groups only")
        if not 0 <= refresh_layer < shape.n_layer:
            raise ValueError("refresh_layer must be one of the model's layers")
        # A draft segment's length is (count - 1) * 16 + last_page_len: the row's current
        # (partial) page must be the last entry of every selection, which only a forced
        # recent page guarantees.
        if recent_pages < 1:
            raise ValueError("recent_pages must be >= 1 (the current page ends every draft list)")
        # The refresh layer scores pages of whole rows; a row cut into query tiles has none.
        if np.any(ql * (shape.n_head // shape.n_local_heads) > 48):
            raise ValueError("q_len * (n_head / n_local_heads) must be at most 48 for every row")
        if caches.shape[1:] != (caches.shape[1], 2, PAGE, shape.n_local_heads, shape.head_dim) \
                or caches.shape[0] != shape.n_layer or caches.dtype != torch.bfloat16:
            raise ValueError("caches must be [n_layer, P, 2, 16, H_kv, 128] bf16")
        B, H = ctx.shape[0], shape.n_local_heads
        self.batch, self.heads = B, H
        self.ctx_len, self.q_len, self.is_draft = ctx, ql, dr
        self.budget, self.refresh_layer, self.recent_pages = int(budget), int(refresh_layer), int(recent_pages)
        self.num_pages_host = (ctx + PAGE - 1) // PAGE
        self.last_host = (ctx - 1) % PAGE + 1
        table = block_table.to(dev, torch.int32).contiguous()
        if table.dim() != 2 or table.shape[0] != B or table.shape[1] < int(self.num_pages_host.max()):
            raise ValueError("block_table must be [B, >= max pages]")
        tab_host = table.cpu()
        if int(tab_host.min()) < 0 or int(tab_host.max()) >= caches.shape[1]:
            raise ValueError("block_table holds pages outside the pool")
        self.block_table = table
        self.T = T = int(ql.sum())
        as_dev = lambda a, dt=torch.int32: torch.from_numpy(np.ascontiguousarray(a)).to(dev, dt)

        # row metadata
        qo = np.zeros(B + 1, dtype=np.int64)
        qo[1:] = np.cumsum(ql)
        self.qo_host = torch.from_numpy(qo.astype(np.int32))
        self.qo_indptr = as_dev(qo)
        self.offsets = as_dev(ctx - ql)
        self.mode_flags = as_dev(np.where(dr, DRAFT_MODE, VERIFY_MODE))
        self.all_verify = torch.full((B,), VERIFY_MODE, dtype=torch.int32, device=dev)
        self.num_pages = as_dev(self.num_pages_host)
        self.last_page_len = as_dev(self.last_host)

        # full row lists: the append, and the refresh layer's attention
        full_ptr = np.zeros(B + 1, dtype=np.int64)
        full_ptr[1:] = np.cumsum(self.num_pages_host)
        self.full_indptr = torch.zeros(B + 1, dtype=torch.int32, device=dev)
        self.full_indices = torch.zeros(max(int(full_ptr[-1]), 1), dtype=torch.int32, device=dev)
        self.full_indptr_host = torch.from_numpy(full_ptr.astype(np.int32))
        self.full_kv_len_host = torch.from_numpy(ctx.astype(np.int32))

        # per-(row, kv head) lists of the other layers: a list per head for draft rows,
        # one shared list per verify row (segment starts as build_head_page_lists lays them out)
        cnt = np.where(dr, np.minimum(self.budget, self.num_pages_host), self.num_pages_host)
        seg_start = np.zeros((B, H), dtype=np.int64)
        pos = 0
        for b in range(B):
            if dr[b]:
                seg_start[b] = pos + cnt[b] * np.arange(H)
                pos += int(cnt[b]) * H
            else:
                seg_start[b] = pos
                pos += int(cnt[b])
        self.mixed_indptr = torch.zeros(B * H + 1, dtype=torch.int32, device=dev)
        self.mixed_indices = torch.zeros(max(pos, 1), dtype=torch.int32, device=dev)
        self.seg_start_host = torch.from_numpy(seg_start.reshape(-1).astype(np.int32))
        self.seg_pages_host = torch.from_numpy(np.repeat(cnt, H).astype(np.int32))
        self.mixed_kv_len_host = torch.from_numpy(np.repeat((cnt - 1) * PAGE + self.last_host, H).astype(np.int32))
        self.draft_counts_host = cnt

        self.selector = KeyMeanPageSelector(B, H, table.shape[1], self.budget, L=self.recent_pages, device=dev,
                                            order="logical")
        # before the first refresh: every draft segment lists the row's last `budget` pages
        init_sel = np.zeros((B, H, self.budget), dtype=np.int32)
        init_cnt = np.zeros((B, H), dtype=np.int32)
        for b in range(B):
            n = int(self.num_pages_host[b])
            c = min(self.budget, n)
            init_sel[b, :, :c] = tab_host[b, n - c : n].numpy()
            init_cnt[b, :] = c
        self.selector.selected.copy_(torch.from_numpy(init_sel))
        self.selector.counts.copy_(torch.from_numpy(init_cnt))
        self.selector.page_scores.zero_()  # verify rows' segments are ranked too (their lists are unused)

        ws = torch.empty(1, device=dev)
        dump_args = None
        if selector == "first_last":
            # the first/last dump of the refresh layer and the reference selector over it
            W = table.shape[1]
            self.kv_stride = W * PAGE  # a multiple of the kernel's KV tile (compute_max_cta_tile_kv)
            self.dump = torch.full((B * shape.n_head * 2 * self.kv_stride,), float("-inf"), dtype=torch.float16,
                                   device=dev)
            self.lse_buf = torch.zeros(self.T, shape.n_head, dtype=torch.float32, device=dev)
            self.fl_selector = PageSelectorFirstLastAvg(
                max_batch_size=B, pages_per_slot=W, subset_cache_size=self.budget, L=self.recent_pages,
                n_heads=shape.n_head, page_size=PAGE, max_seq_length=W * PAGE, device=dev, bsz=B,
                dec_len=int(ql.max()), head_dim=shape.head_dim, kv_stride=self.kv_stride, order="logical")
            rcnt = np.where(dr, np.minimum(self.budget, self.num_pages_host), self.num_pages_host)
            rptr = np.zeros(B + 1, dtype=np.int64)
            rptr[1:] = np.cumsum(rcnt)
            self.row_indptr = torch.zeros(B + 1, dtype=torch.int32, device=dev)
            self.row_indices = torch.zeros(max(int(rptr[-1]), 1), dtype=torch.int32, device=dev)
            self.row_indptr_host = torch.from_numpy(rptr.astype(np.int32))
            self.row_kv_len_host = torch.from_numpy(((rcnt - 1) * PAGE + self.last_host).astype(np.int32))
            self.row_counts_host = rcnt
            # before the first selection: every draft row lists its last `budget` pages
            self.fl_selector._selected_buf[:B].copy_(self.selector.selected[:, 0])
            self.fl_selector._valid_counts_buf[:B].copy_(self.selector.counts[:, 0])
            self.fl_selected = self.fl_selector._selected_buf[:B, : self.budget]
            self.fl_valid = self.fl_selector._valid_counts_buf[:B]
            dump_args = build_holistic_dump_jit_args(torch.bfloat16, shape.head_dim, dump_kind="first_last_compact",
                                                     dump_buffer_dtype=torch.float16)
        self.refresh_wrapper = HolisticAttentionWrapper(ws, "NHD", jit_args=dump_args, waves_per_cu=waves_per_cu)
        self.mixed_wrapper = HolisticAttentionWrapper(ws, "NHD", waves_per_cu=waves_per_cu)
        self.rope = RopeConfig(rope_theta=shape.rope_base)

        # activations
        bf = torch.bfloat16
        self.tokens = tokens.to(dev, torch.int64).contiguous() if tokens is not None else torch.randint(
            0, shape.vocab_size, (T,), generator=torch.Generator(device=dev).manual_seed(seed + 9), device=dev)
        if self.tokens.numel() != T:
            raise ValueError("tokens must hold one id per new token")
        self.x = torch.empty(T, shape.dim, dtype=bf, device=dev)
        self.a = torch.empty(T, shape.dim, dtype=bf, device=dev)
        # q of attention_only (the forward's projections are fresh tensors)
        self.qkv = torch.empty(T, shape.q_size + 2 * shape.kv_size, dtype=bf, device=dev).normal_()
        self.y = torch.empty(T, shape.n_head, shape.head_dim, dtype=bf, device=dev)
        self.act = torch.empty(T, shape.intermediate_size, dtype=bf, device=dev)
        self.ids = torch.zeros(T, dtype=torch.int64, device=dev)
        self.logits = None

        self.build_lists()
        # plan() once (the wrappers' module set-up, as the reference requires before plan_host)
        for wr in (self.refresh_wrapper, self.mixed_wrapper):
            wr.plan(self.qo_indptr, self.full_indptr, self.full_indices, self.last_page_len, shape.n_head,
                    shape.n_local_heads, 128, PAGE, causal=True)
        self.plan()

    # -------------------------------------------------------------- per step
    def plan(self) -> None:
        """Host planning of both attention plans (``plan_host``, no device sync)."""
        s = self.shape
        self.refresh_wrapper.plan_host(self.qo_host, self.full_indptr_host, self.full_kv_len_host, self.full_indices,
                                       s.n_head, s.n_local_heads, 128, PAGE, causal=True)
        if self.selector_kind == "first_last":
            # a draft row keeps min(budget, pages) pages (draft_percent=None), so the plan
            # needs no device readback of the selector's counts
            self.mixed_wrapper.plan_host(self.qo_host, self.row_indptr_host, self.row_kv_len_host, self.row_indices,
                                         s.n_head, s.n_local_heads, 128, PAGE, causal=True)
        else:
            self.mixed_wrapper.plan_segments(self.qo_host, self.seg_start_host, self.seg_pages_host,
                                             self.mixed_kv_len_host, self.mixed_indices, s.n_head, s.n_local_heads,
                                             128, PAGE, causal=True)

    def build_lists(self) -> None:
        """Device page lists: the full row lists and the draft lists from the current selection."""
        self._full_lists()
        if self.selector_kind == "first_last":
            self._row_lists()
        else:
            self._head_lists()

    def _row_lists(self) -> None:
        build_unified_indices(self.mode_flags, self.fl_selected, self.block_table, self.fl_valid, self.num_pages,
                              self.row_indices, self.row_indptr)

    def select_first_last(self) -> None:
        """The reference's step-preparation replan (base.py:580-667,1200-1256): select every
        row's pages from the last refresh layer's dump and LSE, then rebuild the row lists."""
        self.fl_selector.select(self.dump, self.lse_buf, self.num_pages, self.block_table, self.qo_indptr)
        self._row_lists()

    def _full_lists(self) -> None:
        build_unified_indices(self.all_verify, self.block_table, self.block_table, self.num_pages, self.num_pages,
                              self.full_indices, self.full_indptr)

    def _head_lists(self) -> None:
        B = self.batch
        build_head_page_lists(self.mode_flags, self.selector.selected[:B], self.selector.counts[:B],
                              self.block_table, self.num_pages, self.mixed_indices, self.mixed_indptr,
                              share_verify=True)

    def attention(self, layer: int, q: torch.Tensor) -> None:
        cache = self.caches[layer]
        if layer == self.refresh_layer and self.selector_kind == "first_last":
            _, lse = self.refresh_wrapper.run(q, cache, self.dump, self.shape.n_head, self.kv_stride, out=self.y,
                                              return_lse=True)
            self.lse_buf.copy_(lse[: self.T])
        elif layer == self.refresh_layer:
            self.refresh_wrapper.run(q, cache, out=self.y, page_scores=self.selector.page_scores)
            self.selector.select(self.num_pages, self.block_table, self.batch)
            self._head_lists()
        else:
            self.mixed_wrapper.run(q, cache, out=self.y)

    def forward(self, capture: dict | None = None) -> torch.Tensor:
        """One decode step; returns the greedy token ids ``[T]`` (int64, device).

        ``capture`` (a dict, for tests) receives each layer's fused projection
        output before the q/k preparation as ``qkv{layer}``, the attention input q
        (after RoPE) as ``q{layer}``, the attention output as ``y{layer}`` and the
        final hidden state as ``h``."""
        s, w = self.shape, self.w
        T = self.T
        qs, kvs = s.q_size, s.kv_size
        self._full_lists()
        if self.selector_kind == "first_last":
            self.select_first_last()
        torch.index_select(w.tok_embeddings, 0, self.tokens, out=self.x)
        ffn_out = None
        for layer, lw in enumerate(w.layers):
            add_rms_norm(self.x, lw["attention_norm"], self.a, s.norm_eps, delta=ffn_out)
            qkv = F.linear(self.a, lw["wqkv"])
            q = qkv[:, :qs].view(T, s.n_head, s.head_dim)
            k = qkv[:, qs : qs + kvs].view(T, s.n_local_heads, s.head_dim)
            v = qkv[:, qs + kvs :].view(T, s.n_local_heads, s.head_dim)
            if capture is not None:
                capture[f"qkv{layer}"] = qkv.clone()  # q is rewritten in place below
            qk_norm_rope_update_kv(q, k, v, lw["q_norm"], lw["k_norm"], s.norm_eps, self.qo_indptr, self.offsets,
                                   self.caches[layer], self.full_indices, self.full_indptr, self.last_page_len, PAGE,
                                   config=self.rope)
            if capture is not None:
                capture[f"q{layer}"] = q.clone()
            self.attention(layer, q)
            if capture is not None:
                capture[f"y{layer}"] = self.y.clone()
            attn_out = F.linear(self.y.view(T, qs), lw["wo"])
            add_rms_norm(self.x, lw["ffn_norm"], self.a, s.norm_eps, delta=attn_out)
            gate_up = F.linear(self.a, lw["w13"])
            silu_mul(gate_up, self.act)
            ffn_out = F.linear(self.act, lw["w2"])
        add_rms_norm(self.x, w.norm, self.a, s.norm_eps, delta=ffn_out)
        if capture is not None:
            capture["h"] = self.a.clone()
        self.logits = F.linear(self.a, w.output)
        return argmax_rows(self.logits, self.ids)

    def attention_only(self) -> None:
        """The step's attention work alone (for the attention share): both list builds,
        every layer's attention, the refresh selection; q is whatever ``qkv`` holds."""
        s = self.shape
        self._full_lists()
        if self.selector_kind == "first_last":
            self.select_first_last()
        q = self.qkv[:, : s.q_size].view(self.T, s.n_head, s.head_dim)
        for layer in range(s.n_layer):
            self.attention(layer, q)

    # ----------------------------------------------------------- accounting
    def algorithmic_bytes(self) -> dict:
        """HBM bytes one step must move: weights once, every layer's KV reads (per-head
        segments read one head's K and V per page), appends, logits."""
        s = self.shape
        refresh_kv = int(self.ctx_len.sum()) * s.n_local_heads * s.head_dim * 2 * 2
        if self.selector_kind == "first_last":
            mixed_kv = int(self.row_kv_len_host.numpy().astype(np.int64).sum()) * s.n_local_heads * s.head_dim * 2 * 2
        else:
            mixed_kv = int(self.mixed_kv_len_host.numpy().astype(np.int64).sum()) * s.head_dim * 2 * 2
        kv = refresh_kv + (s.n_layer - 1) * mixed_kv
        weights = s.n_layer * self.w.layer_bytes() + self.w.output.numel() * 2 + s.dim * 2
        embed = self.T * s.dim * 2
        append = s.n_layer * self.T * s.kv_size * 2 * 2
        logits = self.T * s.vocab_size * 2
        out = {"kv": kv, "weights": weights, "append": append, "logits": logits}
        if self.selector_kind == "first_last":
            # fp16 dump entries the refresh layer writes (first and last query of each row, one
            # entry when they coincide) and the selector's read of both slots of every page
            slots = np.where(self.q_len > 1, 2, 1)
            out["dump_write"] = int((slots * self.ctx_len).sum()) * s.n_head * 2
            out["dump_read"] = int(self.num_pages_host.sum()) * PAGE * s.n_head * 2 * 2
        out["total"] = sum(out.values())
        return out
