"""CPU oracle for the mixed draft/verify paged-KV attention path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (``aspire_amd``)
imports this package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker or as the
timed CPU baseline, never as a fallback for the HIP path.

Each module restates one piece of the reference semantics on the CPU and cites
the reference ``file:line`` it follows (paths relative to the reference
repository root, e.g. ``aspire/attention/kv_ops.py``):

``append``      paged KV append (integer positions + byte copy), numpy.
``page_list``   mixed draft/verify page-list build, numpy.
``attention``   paged attention with causal masking, GQA, base-2 LSE and the
                first/last logits dump, torch fp32 (optionally fp64) on CPU.
``merge``       split-KV (o, lse) merge, torch fp32.
``select``      the reference first/last page selector (R) and the per-KV-head
                key-mean selector (B), torch on CPU.
``plan``        the host plan-array formulas (qo/kv indptr, kv_len).

How each function is pinned (what would catch a dropped term, a wrong index
or a transposed operand) is stated in that function's docstring and in the
tests that check it; a function without such a check says "parity unpinned".
"""
