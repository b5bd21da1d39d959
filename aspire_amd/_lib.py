"""ctypes binding of libaspire_hip.so (the C ABI declared in include/aspire_hip.h).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already loaded (both use the ``libamdhip64.so.7`` soname). There is no CPU or
PyTorch fallback: if the library is missing every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

# ASPIRE_HIP_LIB selects another build of the same library (a compile-time kernel variant made
# with ``build.py --define ... --out ...``), for A/B measurements.
LIB_PATH = Path(os.environ.get("ASPIRE_HIP_LIB") or Path(__file__).resolve().parent / "libaspire_hip.so").resolve()

ASPIRE_OK = 0
ASPIRE_ERR_INVALID = 1
ASPIRE_ERR_CAPACITY = 2
ASPIRE_ERR_HIP = 3

EXPORTED = (
    "aspire_last_error",
    "aspire_build_info",
    "aspire_max_kv_tile",
    "aspire_paged_kv_append",
    "aspire_build_mixed_page_list",
    "aspire_plan_layout_init",
    "aspire_plan_build",
    "aspire_plan_upload",
    "aspire_attention_run",
    "aspire_merge_states",
    "aspire_select_first_last_scores",
    "aspire_select_topk",
    "aspire_host_plan_reset",
    "aspire_host_plan_step",
    "aspire_qk_norm_rope_append",
    "aspire_rope_frequencies",
    "aspire_build_head_page_lists",
    "aspire_plan_build_segments",
    "aspire_add_rms_norm",
    "aspire_silu_mul",
    "aspire_argmax_rows",
    "aspire_attention_run_static",
    "aspire_topk_candidates",
    "aspire_logits_pipe",
    "aspire_sampling_from_probs",
    "aspire_chain_speculative_sampling",
    "aspire_verify_topk_speculation",
    "aspire_prefill_block_tokens",
    "aspire_prefill_run",
    "aspire_bandwidth_probe",
)

# Bytes of the static device scratch behind aspire_attention_run_static (ASPIRE_STATIC_SCRATCH_BYTES).
STATIC_SCRATCH_BYTES = 64 << 20


class PlanLayout(ctypes.Structure):
    _fields_ = [
        ("num_waves", ctypes.c_int32),
        ("max_items", ctypes.c_int32),
        ("max_merge", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("partial_rows_cap", ctypes.c_int64),
        ("int_ws_bytes", ctypes.c_int64),
        ("float_ws_bytes", ctypes.c_int64),
    ]


class PlanInfo(ctypes.Structure):
    _fields_ = [
        ("num_items", ctypes.c_int32 * 3),
        ("num_merge", ctypes.c_int32),
        ("partial_rows", ctypes.c_int64),
        ("num_segments", ctypes.c_int32),
        ("max_rows", ctypes.c_int32),
        ("total_pages", ctypes.c_int64),
        ("live_bytes", ctypes.c_int64),
        ("split_rows", ctypes.c_int32),
    ]


class AttentionArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_stride_t", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("kv_cache", ctypes.c_void_p), ("cache_stride_p", ctypes.c_int64),
        ("cache_stride_kv", ctypes.c_int64), ("cache_stride_t", ctypes.c_int64),
        ("cache_stride_h", ctypes.c_int64),
        ("kv_indices", ctypes.c_void_p),
        ("out", ctypes.c_void_p), ("out_stride_t", ctypes.c_int64), ("out_stride_h", ctypes.c_int64),
        ("lse", ctypes.c_void_p),
        ("plan_dev", ctypes.c_void_p),
        ("float_ws", ctypes.c_void_p),
        ("num_qo_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("page_size", ctypes.c_int32),
        ("sm_scale", ctypes.c_float), ("causal", ctypes.c_int32),
        ("class_mask", ctypes.c_int32), ("launch_merge", ctypes.c_int32),
        ("dump", ctypes.c_void_p), ("dump_kind", ctypes.c_int32), ("dump_dtype", ctypes.c_int32),
        ("dump_kv_stride", ctypes.c_int64), ("dump_num_heads", ctypes.c_int32),
        ("dump_mode_flags", ctypes.c_void_p),
        ("page_scores", ctypes.c_void_p), ("page_score_stride", ctypes.c_int64),
        ("partial_nt", ctypes.c_int32),
    ]


class PrefillArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_stride_t", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("kv_cache", ctypes.c_void_p), ("cache_stride_p", ctypes.c_int64), ("cache_stride_kv", ctypes.c_int64),
        ("cache_stride_t", ctypes.c_int64), ("cache_stride_h", ctypes.c_int64),
        ("kv_indices", ctypes.c_void_p), ("kv_indptr", ctypes.c_void_p), ("kv_last_page_len", ctypes.c_void_p),
        ("qo_indptr", ctypes.c_void_p), ("block_indptr", ctypes.c_void_p),
        ("num_rows", ctypes.c_int32), ("total_blocks", ctypes.c_int32), ("block_tokens", ctypes.c_int32),
        ("out", ctypes.c_void_p), ("out_stride_t", ctypes.c_int64), ("out_stride_h", ctypes.c_int64),
        ("lse", ctypes.c_void_p),
        ("num_qo_heads", ctypes.c_int32), ("num_kv_heads", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32), ("sm_scale", ctypes.c_float), ("causal", ctypes.c_int32),
    ]


_lock = threading.Lock()
class HostPlanConfig(ctypes.Structure):
    _fields_ = [
        ("page_size", ctypes.c_int32), ("max_batch", ctypes.c_int32), ("draft_kind", ctypes.c_int32),
        ("full_kind", ctypes.c_int32), ("subset_cache_size", ctypes.c_int32), ("table_width", ctypes.c_int32),
        ("min_draft_pages", ctypes.c_int32), ("draft_percent", ctypes.c_float), ("valid_floor_l", ctypes.c_int32),
        ("pages_per_slot", ctypes.c_int32),
    ]


class HostPlanStateC(ctypes.Structure):
    _fields_ = [("draft_num_pages", ctypes.c_void_p), ("prev_verify", ctypes.c_void_p)]


class HostPlanInputs(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32), ("verify", ctypes.c_void_p), ("finished", ctypes.c_void_p),
        ("draft_counts", ctypes.c_void_p), ("seq_lens", ctypes.c_void_p), ("total_tokens", ctypes.c_int64),
        ("bucket_tokens", ctypes.c_int64),
    ]


class HostPlanOutputs(ctypes.Structure):
    _fields_ = [
        ("qo_indptr", ctypes.c_void_p), ("kv_indptr", ctypes.c_void_p), ("kv_len", ctypes.c_void_p),
        ("full_kv_indptr", ctypes.c_void_p), ("full_kv_len", ctypes.c_void_p), ("dec", ctypes.c_void_p),
        ("verify_num_pages", ctypes.c_void_p), ("effective_num_pages", ctypes.c_void_p),
        ("last_page_len", ctypes.c_void_p), ("input_pos", ctypes.c_void_p), ("sample_indices", ctypes.c_void_p),
        ("position_indices", ctypes.c_void_p), ("token_capacity", ctypes.c_int64),
        ("refresh_rows", ctypes.c_void_p), ("spill_rows", ctypes.c_void_p), ("n_refresh", ctypes.c_int32),
        ("n_spill", ctypes.c_int32),
    ]


class RopeArgs(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("q_stride_t", ctypes.c_int64), ("q_stride_h", ctypes.c_int64),
        ("num_qo_heads", ctypes.c_int32),
        ("k", ctypes.c_void_p), ("k_stride_t", ctypes.c_int64), ("k_stride_h", ctypes.c_int64),
        ("num_kv_heads", ctypes.c_int32),
        ("v", ctypes.c_void_p), ("v_stride_t", ctypes.c_int64), ("v_stride_h", ctypes.c_int64),
        ("total_tokens", ctypes.c_int32), ("head_dim", ctypes.c_int32),
        ("q_norm_weight", ctypes.c_void_p), ("k_norm_weight", ctypes.c_void_p), ("norm_eps", ctypes.c_float),
        ("permute", ctypes.c_int32), ("rope_theta", ctypes.c_float), ("rope_scale", ctypes.c_float),
        ("llama31", ctypes.c_int32), ("low_freq_factor", ctypes.c_float), ("high_freq_factor", ctypes.c_float),
        ("old_context_len", ctypes.c_float),
        ("indptr", ctypes.c_void_p), ("offsets", ctypes.c_void_p), ("num_rows", ctypes.c_int32),
        ("kv_cache", ctypes.c_void_p), ("cache_stride_p", ctypes.c_int64), ("cache_stride_kv", ctypes.c_int64),
        ("cache_stride_t", ctypes.c_int64), ("cache_stride_h", ctypes.c_int64), ("page_size", ctypes.c_int32),
        ("kv_page_indices", ctypes.c_void_p), ("kv_page_indptr", ctypes.c_void_p),
        ("kv_last_page_len", ctypes.c_void_p), ("num_seq", ctypes.c_int32), ("write_k", ctypes.c_int32),
    ]


_lib = None


def _declare(lib):
    vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
    lib.aspire_last_error.restype = ctypes.c_char_p
    lib.aspire_build_info.restype = ctypes.c_char_p
    lib.aspire_max_kv_tile.restype = i32
    sigs = {
        "aspire_paged_kv_append": [vp, vp, i64, i64, i64, i64, vp, vp, vp, vp, i32, vp, i64, i64, i64, i64,
                                   i32, i32, i32, i32, vp],
        "aspire_build_mixed_page_list": [vp, i32, vp, i64, i64, vp, i64, i64, vp, vp, i32, vp, i64, vp, i32, vp],
        "aspire_plan_layout_init": [i32, i32, i64, i64, i32, ctypes.POINTER(PlanLayout)],
        "aspire_plan_build": [ctypes.POINTER(PlanLayout), vp, vp, vp, i32, i32, i32, i32, i32, i32, vp, i64,
                              ctypes.POINTER(PlanInfo)],
        "aspire_plan_upload": [ctypes.POINTER(PlanLayout), ctypes.POINTER(PlanInfo), vp, vp, vp],
        "aspire_attention_run": [ctypes.POINTER(PlanLayout), ctypes.POINTER(AttentionArgs), vp],
        "aspire_attention_run_static": [ctypes.POINTER(PlanLayout), ctypes.POINTER(AttentionArgs), vp],
        "aspire_merge_states": [vp, vp, i32, i64, i32, vp, i32, vp, vp],
        "aspire_select_first_last_scores": [vp, i64, i32, i32, i32, vp, i32, vp, vp, vp, i32, i32, f32, vp, i64,
                                            i32, vp],  # ..., scores, score_stride, slots, stream
        "aspire_select_topk": [vp, i64, vp, vp, i32, i32, i32, i32, i32, i32, f32, vp, i64, i32, vp, i64, i32,
                               vp, vp],
        "aspire_host_plan_reset": [ctypes.POINTER(HostPlanConfig), vp, vp, vp, vp, i32],
        "aspire_host_plan_step": [ctypes.POINTER(HostPlanConfig), ctypes.POINTER(HostPlanStateC),
                                  ctypes.POINTER(HostPlanInputs), ctypes.POINTER(HostPlanOutputs)],
        "aspire_qk_norm_rope_append": [ctypes.POINTER(RopeArgs), vp],
        "aspire_rope_frequencies": [i32, f32, f32, i32, f32, f32, f32, vp],
        "aspire_build_head_page_lists": [vp, i32, vp, i64, vp, vp, i64, i64, vp, i32, i32, i32, vp, i64, vp, i32,
                                         vp],
        "aspire_plan_build_segments": [ctypes.POINTER(PlanLayout), vp, vp, vp, vp, i32, i32, i32, i32, i32, vp, i64,
                                       ctypes.POINTER(PlanInfo)],
        "aspire_add_rms_norm": [vp, i64, vp, i64, vp, vp, i64, i32, i32, f32, vp],
        "aspire_silu_mul": [vp, i64, vp, i64, i32, i32, vp],
        "aspire_argmax_rows": [vp, i64, i32, i32, vp, vp],
        "aspire_topk_candidates": [vp, i64, i32, i32, i32, i64, vp, vp, vp],
        "aspire_logits_pipe": [vp, i32, i64, i32, i32, f32, f32, vp, i64, vp],
        "aspire_sampling_from_probs": [vp, i64, i32, i32, vp, vp, vp],
        "aspire_chain_speculative_sampling": [vp, vp, vp, i32, i32, i32, vp, vp, vp, vp, vp],
        "aspire_verify_topk_speculation": [vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp],
        "aspire_prefill_block_tokens": [i32, i32],
        "aspire_prefill_run": [ctypes.POINTER(PrefillArgs), vp],
        "aspire_bandwidth_probe": [i32, vp, i64, vp, i64, i32, i32, vp],
    }
    for name, argtypes in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int


def lib():
    """The loaded library; raises RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python aspire_amd/csrc/build.py` "
                    "(the HIP path has no CPU fallback)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            _declare(handle)
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc == ASPIRE_OK:
        return
    msg = lib().aspire_last_error().decode(errors="replace")
    if rc == ASPIRE_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    """The current HIP stream of ``t``'s device as a ctypes pointer."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_cuda(*tensors: torch.Tensor, what: str) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise RuntimeError(f"{what}: tensors must be on a ROCm GPU (got {t.device}); "
                               "there is no CPU implementation")


def build_info() -> str:
    return lib().aspire_build_info().decode()
