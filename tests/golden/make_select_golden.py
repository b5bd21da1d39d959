"""Write golden vectors for the reference first/last page selector.

Run in the build container only (the reference tree is not on the GPU box):

    python tests/golden/make_select_golden.py /root/reference

It loads ``aspire/backends/page_selector.py`` from the reference checkout by
file path (the module imports only ``math`` and ``torch``), runs
``PageSelectorFirstLastAvg.select`` on seeded CPU inputs, and records the
inputs, the page scores the selector hands to ``_finalize_scores`` and its
outputs in ``select_first_last.npz`` beside this script. Only data is written;
nothing from the reference source is copied.
"""

from __future__ import annotations

import sys

# Loading the reference module must leave nothing in its tree: no __pycache__.
sys.dont_write_bytecode = True

import importlib.util  # noqa: E402
import math  # noqa: E402
from pathlib import Path  # noqa: E402

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def load_reference_selector(ref_root: Path):
    path = ref_root / "aspire" / "backends" / "page_selector.py"
    spec = importlib.util.spec_from_file_location("_ref_page_selector", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


CASES = [
    # name, B, H, page, max_seq, kv_stride, subset, L, draft_percent, min_pages, qlens, num_pages, table
    dict(name="small_fixed", B=4, H=16, page=16, max_seq=256, kv_stride=320, subset=6, L=2,
         draft_percent=None, min_pages=6, qlens=[1, 1, 5, 5], num_pages=[16, 9, 3, 0], table="perm"),
    dict(name="percent", B=3, H=4, page=16, max_seq=2048, kv_stride=2048, subset=12, L=4,
         draft_percent=7.0, min_pages=4, qlens=[3, 1, 6], num_pages=[128, 57, 2], table="arange"),
    dict(name="ties_inf", B=2, H=8, page=16, max_seq=512, kv_stride=576, subset=8, L=1,
         draft_percent=None, min_pages=8, qlens=[2, 1], num_pages=[32, 20], table="arange"),
]


def make_case(ref, c, gen):
    B, H, page, max_seq, kv_stride = c["B"], c["H"], c["page"], c["max_seq"], c["kv_stride"]
    pages_per_slot = max_seq // page
    qlens = torch.tensor(c["qlens"], dtype=torch.int32)
    qo_indptr = torch.zeros(B + 2, dtype=torch.int32)
    qo_indptr[1 : B + 1] = torch.cumsum(qlens, 0)
    qo_indptr[B + 1] = qo_indptr[B]
    T = int(qo_indptr[B])
    # Raw logits ~ N(0, 6^2) in fp16, with -inf for slots never written
    # (past each row's kv_len, and slot 1 of single-query rows).
    dump = (torch.randn(B, H, 2, kv_stride, generator=gen) * 6.0).to(torch.float16)
    num_pages = torch.tensor(c["num_pages"], dtype=torch.int32)
    for b in range(B):
        kv_len = int(num_pages[b]) * page - int(torch.randint(0, page, (1,), generator=gen)) if num_pages[b] > 0 else 0
        dump[b, :, :, kv_len:] = float("-inf")
        if int(qlens[b]) == 1:
            dump[b, :, 1, :] = float("-inf")
    if c["name"] == "ties_inf":
        dump[0, :, :, 40:72] = 0.0  # equal logits -> tied page scores
        dump[1, 3, 0, 100] = float("nan")
        dump[1, 2, 0, 130] = float("inf")
    lse = (torch.randn(max(T, 1), H, generator=gen) * 2.0 + 8.0).to(torch.float32)
    if c["table"] == "perm":
        block_table = torch.randperm(B * pages_per_slot, generator=gen).to(torch.int32).view(B, pages_per_slot)
    else:
        block_table = torch.arange(B * pages_per_slot, dtype=torch.int32).view(B, pages_per_slot)

    sel = ref.PageSelectorFirstLastAvg(
        max_batch_size=B, pages_per_slot=pages_per_slot, subset_cache_size=c["subset"], L=c["L"],
        n_heads=H, page_size=page, max_seq_length=max_seq, device="cpu", bsz=B, dec_len=8,
        head_dim=128, kv_stride=kv_stride, draft_percent=c["draft_percent"], min_draft_pages=c["min_pages"],
    )
    captured = {}
    orig = sel._finalize_scores

    def spy(scores, num_pages_, block_table_):
        captured["scores"] = scores.clone()
        return orig(scores, num_pages_, block_table_)

    sel._finalize_scores = spy
    selected, valid = sel.select(dump.view(-1), lse, num_pages, block_table, qo_indptr)
    prefix = c["name"] + "/"
    return {
        prefix + "dump": dump.view(-1).view(torch.int16).numpy(),
        prefix + "lse": lse.numpy(),
        prefix + "num_pages": num_pages.numpy(),
        prefix + "block_table": block_table.numpy(),
        prefix + "qo_indptr": qo_indptr.numpy(),
        prefix + "scores": captured["scores"].numpy(),
        prefix + "selected": selected.clone().numpy(),
        prefix + "valid": valid.clone().numpy(),
        prefix + "params": np.array(
            [B, H, page, max_seq, kv_stride, c["subset"], c["L"],
             -1 if c["draft_percent"] is None else c["draft_percent"], c["min_pages"]], dtype=np.float64),
    }


def main():
    ref_root = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    ref = load_reference_selector(ref_root)
    gen = torch.Generator().manual_seed(1234)
    arrays = {}
    for c in CASES:
        arrays.update(make_case(ref, c, gen))
    np.savez_compressed(HERE / "select_first_last.npz", case_names=np.array([c["name"] for c in CASES]), **arrays)
    print("wrote", HERE / "select_first_last.npz", "cases:", [c["name"] for c in CASES])


if __name__ == "__main__":
    main()
