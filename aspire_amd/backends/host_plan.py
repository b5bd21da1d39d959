"""Host mirror of the per-step attention-plan arrays, backed by native code.

Replaces ``aspire/backends/host_plan.py`` with the same names and behaviour:
``HostPlanConfig`` (host_plan.py:30-57) and ``HostPlanState`` (59-306) with
``reset_all`` / ``reset_slots`` / ``build_step``. The per-step bookkeeping
(decode tokens, cache lengths, draft-table page counts per refresh family,
spill and refresh rows, the rendered ``qo_indptr`` / ``kv_indptr`` /
``kv_len`` and the dump wrapper's full-context arrays) runs in C++
(``aspire_host_plan_step``); this class owns the state and the output buffers
and returns them in the reference's dict layout. Host memory only.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from aspire_amd import _lib

_DRAFT_KINDS = {"replan": 0, "sink_recent": 1, "gated": 2}
_FULL_KINDS = {None: 0, "mirror": 1, "effective_full": 2}


@dataclass(frozen=True)
class HostPlanConfig:
    """Static settings of the attention backend (page size, batch capacity, draft-table
    refresh family, dump-wrapper layout, selection budgets) that fix how each step's
    plan arrays are rendered."""

    page_size: int
    max_batch: int
    draft_kind: str
    full_kind: str | None
    subset_cache_size: int
    table_width: int
    min_draft_pages: int | None
    draft_percent: float | None
    valid_floor_l: int
    pages_per_slot: int = 0

    def to_c(self) -> _lib.HostPlanConfig:
        if self.draft_kind not in _DRAFT_KINDS:
            raise ValueError(f"unknown draft_kind {self.draft_kind!r}")
        if self.full_kind not in _FULL_KINDS:
            raise ValueError(f"unknown full_kind {self.full_kind!r}")
        return _lib.HostPlanConfig(
            page_size=self.page_size, max_batch=self.max_batch, draft_kind=_DRAFT_KINDS[self.draft_kind],
            full_kind=_FULL_KINDS[self.full_kind], subset_cache_size=self.subset_cache_size,
            table_width=self.table_width,
            min_draft_pages=-1 if self.min_draft_pages is None else int(self.min_draft_pages),
            draft_percent=-1.0 if self.draft_percent is None else float(self.draft_percent),
            valid_floor_l=self.valid_floor_l, pages_per_slot=self.pages_per_slot)


def _p(a) -> ctypes.c_void_p:
    if isinstance(a, torch.Tensor):
        return ctypes.c_void_p(a.data_ptr())
    return ctypes.c_void_p(a.ctypes.data)


class HostPlanState:
    """Per-row length and page-count state kept on the host, advanced once per decode
    step so the plan arrays never need a device readback (host_plan.py:59-306).

    The plan tensors and the per-row / per-token arrays ``build_step`` returns
    are views of buffers this object owns (allocated once, as the reference
    allocates its plan tensors once): they hold the last step's values until
    the next ``build_step``.
    """

    def __init__(self, config: HostPlanConfig):
        self.config = config
        self._cfg = config.to_c()
        mb = config.max_batch
        self.draft_num_pages = np.zeros(mb, dtype=np.int64)
        self._prev_verify = np.zeros(mb, dtype=np.bool_)
        self.qo_indptr = torch.zeros(mb + 2, dtype=torch.int32)
        self.kv_indptr = torch.zeros(mb + 2, dtype=torch.int32)
        self.kv_len = torch.zeros(mb + 1, dtype=torch.int32)
        self.full_kv_indptr = torch.zeros(mb + 2, dtype=torch.int32)
        self.full_kv_len = torch.zeros(mb + 1, dtype=torch.int32)
        self._state = _lib.HostPlanStateC(_p(self.draft_num_pages), _p(self._prev_verify.view(np.uint8)))
        self._rows = {k: np.zeros(mb, dtype=np.int64)
                      for k in ("dec", "verify_num_pages", "effective_num_pages", "last_page_len", "input_pos",
                                "refresh_rows", "spill_rows")}
        self._ins = _lib.HostPlanInputs()
        self._outs = _lib.HostPlanOutputs()
        full = config.full_kind == "effective_full"
        o = self._outs
        o.qo_indptr, o.kv_indptr, o.kv_len = _p(self.qo_indptr), _p(self.kv_indptr), _p(self.kv_len)
        o.full_kv_indptr = _p(self.full_kv_indptr) if full else None
        o.full_kv_len = _p(self.full_kv_len) if full else None
        for k in ("dec", "verify_num_pages", "effective_num_pages", "last_page_len", "input_pos", "refresh_rows",
                  "spill_rows"):
            setattr(o, k, _p(self._rows[k]))
        self._reserve_tokens(16 * max(mb, 1))
        self._fn = _lib.lib().aspire_host_plan_step
        self._args = (ctypes.byref(self._cfg), ctypes.byref(self._state), ctypes.byref(self._ins),
                      ctypes.byref(self._outs))

    def _reserve_tokens(self, n: int) -> None:
        self._sample = np.zeros(n, dtype=np.int64)
        self._position = np.zeros(n, dtype=np.int64)
        self._outs.sample_indices, self._outs.position_indices = _p(self._sample), _p(self._position)
        self._outs.token_capacity = n

    def reset_all(self, seq_lens) -> None:
        lens = np.ascontiguousarray(seq_lens, dtype=np.int64)
        _lib.check(_lib.lib().aspire_host_plan_reset(ctypes.byref(self._cfg), _p(self.draft_num_pages),
                                                     _p(self._prev_verify.view(np.uint8)), None, _p(lens),
                                                     int(lens.size)), "HostPlanState.reset_all")

    def reset_slots(self, slot_ids, seq_lens) -> None:
        ids = np.ascontiguousarray(slot_ids, dtype=np.int64)
        lens = np.ascontiguousarray(seq_lens, dtype=np.int64)
        if ids.size != lens.size:
            raise ValueError("slot_ids and seq_lens differ in length")
        _lib.check(_lib.lib().aspire_host_plan_reset(ctypes.byref(self._cfg), _p(self.draft_num_pages),
                                                     _p(self._prev_verify.view(np.uint8)), _p(ids), _p(lens),
                                                     int(ids.size)), "HostPlanState.reset_slots")

    def build_step(self, *, verify: np.ndarray, finished: np.ndarray, draft_counts: np.ndarray,
                   seq_lens: np.ndarray, total_tokens: int, bucket_tokens: int) -> dict:
        cfg = self.config
        mb = int(verify.shape[0])
        v = np.ascontiguousarray(verify, dtype=np.bool_)
        f = np.ascontiguousarray(finished, dtype=np.bool_)
        d = np.ascontiguousarray(draft_counts, dtype=np.int64)
        s = np.ascontiguousarray(seq_lens, dtype=np.int64)
        ntok = max(int(total_tokens), 0)
        if ntok > self._outs.token_capacity:
            self._reserve_tokens(2 * ntok)
        ins = self._ins
        ins.batch, ins.total_tokens, ins.bucket_tokens = mb, int(total_tokens), int(bucket_tokens)
        ins.verify, ins.finished = v.ctypes.data, f.ctypes.data
        ins.draft_counts, ins.seq_lens = d.ctypes.data, s.ctypes.data
        if self._fn(*self._args) != _lib.ASPIRE_OK:
            # the reference raises RuntimeError for a diverged mirror (host_plan.py:240-244)
            raise RuntimeError(_lib.lib().aspire_last_error().decode(errors="replace"))
        r = self._rows
        result = {
            "qo_indptr": self.qo_indptr,
            "kv_indptr": self.kv_indptr,
            "kv_len": self.kv_len,
            "full_qo_indptr": None,
            "full_kv_indptr": None,
            "full_kv_len": None,
            "spill_rows": r["spill_rows"][: self._outs.n_spill],
            "refresh_rows": r["refresh_rows"][: self._outs.n_refresh],
            "draft_num_pages": self.draft_num_pages,
            "dec": r["dec"][:mb],
            "verify_num_pages": r["verify_num_pages"][:mb],
            "effective_num_pages": r["effective_num_pages"][:mb],
            "last_page_len": r["last_page_len"][:mb],
            "input_pos": r["input_pos"][:mb],
            "sample_indices": self._sample[:ntok],
            "position_indices": self._position[:ntok],
        }
        if cfg.full_kind == "mirror":
            result["full_qo_indptr"] = self.qo_indptr
            result["full_kv_indptr"] = self.kv_indptr
            result["full_kv_len"] = self.kv_len
        elif cfg.full_kind == "effective_full":
            result["full_qo_indptr"] = self.qo_indptr
            result["full_kv_indptr"] = self.full_kv_indptr
            result["full_kv_len"] = self.full_kv_len
        return result


__all__ = ["HostPlanConfig", "HostPlanState"]
