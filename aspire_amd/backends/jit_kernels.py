"""Attention-weight dump variants (HIP implementation).

Drop-in for ``aspire/backends/jit_kernels.py``. The reference generates CUDA
structs (logits-transform callbacks) that FlashInfer JIT-compiles into its
attention kernel (jit_kernels.py:74-96,179-256). Here the dump is a compile-time
epilogue of the HIP attention kernel, so ``build_dump_struct`` returns a
``DumpVariant`` description instead of source text, and the argument lists keep
the reference's shape so call sites are unchanged.

Dump semantics (the kernel's, identical to jit_kernels.py:182-193,247-256):
``first_last_compact`` writes ``fp16(q.k)`` of query 0 to slot 0 and of query
``qo_len - 1`` to slot 1 at ``((b*num_heads + h)*2 + slot)*kv_stride + kv_idx``;
``last_token`` writes query ``qo_len - 1`` at ``(b*num_heads + h)*kv_stride +
kv_idx``; ``noop`` writes nothing. ``use_mode_flags`` skips rows whose flag is
0. Unlike the reference callback, the kernel keeps the ``kv_idx < kv_len``
guard, so the stride needs no tile padding and nothing past kv_len is written.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

_BASE_TENSOR_NAMES = ["attention_weights"]
_FA2_SCALAR_NAMES = ["sm_scale", "num_heads", "jit_kv_stride"]
_FA2_SCALAR_TYPES = ["double", "int64_t", "int64_t"]
_HOLISTIC_SCALAR_NAMES = ["num_heads", "jit_kv_stride"]
_HOLISTIC_SCALAR_TYPES = ["int64_t", "int64_t"]

DUMP_KINDS = ("noop", "last_token", "first_last_compact")
_TYPE_NAMES = {torch.float16: "half", torch.float32: "float", torch.bfloat16: "nv_bfloat16"}


@dataclass(frozen=True)
class DumpVariant:
    """What the attention kernel's dump epilogue writes (replaces the JIT struct source)."""

    backend: str
    kind: str
    class_name: str
    use_mode_flags: bool
    attn_type: str

    @property
    def kernel_kind(self) -> int:
        """Code passed to aspire_attention_run: 0 none, 1 last_token, 2 first_last."""
        return {"noop": 0, "last_token": 1, "first_last_compact": 2}[self.kind]

    @property
    def slots(self) -> int:
        return 2 if self.kind == "first_last_compact" else 1


def build_dump_struct(backend: str, dump_kind: str, class_name: str, use_mode_flags: bool = False,
                      attn_type: str = "float") -> DumpVariant:
    """Describe a dump variant (reference: jit_kernels.py:271-332)."""
    if backend not in ("fa2", "fa3", "holistic", "hip"):
        raise ValueError(f"Unknown backend={backend!r}")
    if dump_kind not in DUMP_KINDS:
        raise ValueError(f"Unknown dump_kind={dump_kind!r}")
    if attn_type not in ("half", "float"):
        raise ValueError(f"dump buffers must be fp16 or fp32, got {attn_type!r}")
    use_mode = use_mode_flags and dump_kind != "noop"
    return DumpVariant(backend, dump_kind, class_name, use_mode, attn_type)


def _scalar_spec(backend: str):
    if backend == "holistic":
        return list(_HOLISTIC_SCALAR_NAMES), list(_HOLISTIC_SCALAR_TYPES)
    return list(_FA2_SCALAR_NAMES), list(_FA2_SCALAR_TYPES)


def _type_name(dtype: torch.dtype) -> str:
    try:
        return _TYPE_NAMES[dtype]
    except KeyError as exc:
        raise ValueError(f"unsupported dump buffer dtype {dtype}") from exc


def build_dump_jit_args(backend: str, dtype: torch.dtype, head_dim: int, dump_kind: str = "last_token",
                        class_name: str = "BatchDumpAttentionWeights",
                        op_name: str = "batch_prefill_dump_attention_weights", use_mode_flags: bool = False,
                        dump_buffer_dtype: torch.dtype = torch.float32) -> list:
    """Argument list in the reference's shape (jit_kernels.py:357-392); entry 12 is a DumpVariant."""
    backend_key = "fa3" if backend == "fa3" else "fa2"
    scalar_names, scalar_types = _scalar_spec(backend_key)
    attn_type = _type_name(dump_buffer_dtype)
    spec = build_dump_struct(backend_key, dump_kind, class_name, use_mode_flags, attn_type=attn_type)
    tensor_names = list(_BASE_TENSOR_NAMES)
    tensor_types = [attn_type]
    if use_mode_flags and dump_kind != "noop":
        tensor_names.append("mode_flags")
        tensor_types.append("int32_t")
    return [op_name, dtype, dtype, dtype, torch.int32, head_dim, head_dim, tensor_names, tensor_types,
            scalar_names, scalar_types, class_name, spec]
