"""Logits processing on the HIP path: drop-in for the ``flashinfer.logits_processor`` pieces
the reference composes (aspire/models/sparse_draft_runner.py:527-554).

``LogitsPipe([Temperature(), Softmax(), TopP()])(values, temperature=..., top_p=...)`` runs
one kernel (``aspire_logits_pipe``): fp32 ``softmax(values / temperature)`` and top-p
renormalisation per row. ``define_logit_process_op`` registers ``mylib::logit_process``
around a pipe, as ``_define_logit_op`` does, with the fake (meta) implementation
torch.compile traces through.
"""

from __future__ import annotations

import torch

from aspire_amd import _lib


class Temperature:
    """Divide the values by ``temperature`` (a keyword of the pipe call)."""


class Softmax:
    """Softmax over the last dimension, in fp32."""


class TopP:
    """Top-p renormalisation with ``top_p`` (a keyword of the pipe call)."""


_ORDER = (Temperature, Softmax, TopP)


class LogitsPipe:
    """A sequence of the ops above; Softmax is required, Temperature may precede it and TopP
    follow it (the compositions the reference builds)."""

    def __init__(self, ops):
        kinds = [type(op) for op in ops]
        if Softmax not in kinds:
            raise ValueError("LogitsPipe needs a Softmax")
        idx = [_ORDER.index(k) if k in _ORDER else -1 for k in kinds]
        if -1 in idx or idx != sorted(idx) or len(set(idx)) != len(idx):
            raise ValueError("supported pipes: [Temperature()], Softmax(), [TopP()] in that order")
        self.ops = list(ops)
        self._temperature = Temperature in kinds
        self._top_p = TopP in kinds

    def __call__(self, values: torch.Tensor, temperature: float | None = None, top_p: float | None = None):
        if self._temperature and temperature is None:
            raise ValueError("this pipe applies Temperature: pass temperature=")
        if self._top_p and top_p is None:
            raise ValueError("this pipe applies TopP: pass top_p=")
        _lib.require_cuda(values, what="LogitsPipe")
        if values.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("values must be bf16 or fp32")
        shape = values.shape
        v = values.reshape(-1, shape[-1])
        if v.stride(-1) != 1:
            v = v.contiguous()
        rows, width = v.shape
        probs = torch.empty(rows, width, dtype=torch.float32, device=values.device)
        rc = _lib.lib().aspire_logits_pipe(
            _lib.ptr(v), 1 if v.dtype == torch.float32 else 0, v.stride(0), rows, width,
            float(temperature) if self._temperature else 0.0, float(top_p) if self._top_p else 0.0,
            _lib.ptr(probs), probs.stride(0), _lib.stream_of(values))
        _lib.check(rc, "LogitsPipe")
        return probs.view(shape)


def define_logit_process_op(pipe: LogitsPipe, kwargs: dict):
    """Register ``mylib::logit_process(Tensor vals) -> Tensor`` running ``pipe(vals, **kwargs)``
    (sparse_draft_runner.py:527-537); the fake implementation returns an fp32 tensor like vals."""
    torch.library.define("mylib::logit_process", "(Tensor vals) -> Tensor")

    @torch.library.impl("mylib::logit_process", "cuda")
    def _logit_process(vals):
        return pipe(vals, **kwargs)

    @torch.library.register_fake("mylib::logit_process")
    def _logit_process_fake(vals):
        return torch.empty_like(vals, dtype=torch.float32)

    return torch.ops.mylib.logit_process


def build_logits_pipe(temperature: float = 0, top_p: float = 0):
    """The pipe and keywords ``set_logit_processing`` builds: Temperature when temperature > 0,
    Softmax, TopP when top_p > 0."""
    ops, kwargs = [], {}
    if temperature > 0:
        ops.append(Temperature())
        kwargs["temperature"] = temperature
    ops.append(Softmax())
    if top_p > 0:
        ops.append(TopP())
        kwargs["top_p"] = top_p
    return LogitsPipe(ops), kwargs


__all__ = ["LogitsPipe", "Temperature", "Softmax", "TopP", "define_logit_process_op", "build_logits_pipe"]
