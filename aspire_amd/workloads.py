"""Seeded synthetic inputs for one mixed draft/verify attention layer.

Shapes follow BASELINE.json's configs (page size 16, head_dim 128, bf16):

* config 0 - Qwen3-1.7B shape (16 q / 8 kv heads), batch 4, every context 4096
  tokens, a 1024-page pool in random-permutation order; rows 0-1 draft
  (q_len 1 over a 64-page selection), rows 2-3 verify (q_len 5, full cache);
* config 1 - Qwen3-8B shape (32 / 8 heads), batch 32, every context 32768
  tokens, a 65536-page pool in random order; rows 0-15 draft (q_len 1 over 128
  selected pages), rows 16-31 verify (q_len 4);
* config 2 - Qwen3-8B refresh layer: batch 64, contexts uniform in
  [8192, 32768], every row a single query over its full cache;
* config 4 - DeepSeek-R1-Distill-Llama-8B shape (32 / 8 heads), batch 16,
  contexts uniform in [65536, 131072]; a fraction f of the rows draft (q_len 1
  over a 256-page selection), the rest verify with q_len uniform in {2..9}.

K, V and Q are N(0, 1); every (page, kv head) adds one N(0, 0.5^2) scalar to
all 16 of its keys so page scores separate. A row's context length is its KV
length at attention time, after the append: the new tokens occupy its last
q_len positions. Draft rows attend a selection of their pages that always ends
with the current (last) page, listed in ascending logical order.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

PAGE = 16
HEAD_DIM = 128


@dataclass
class MixedStep:
    """One layer's inputs: cache, queries, new K/V and the mixed page lists."""

    hq: int
    hkv: int
    cache: torch.Tensor            # [P, 2, 16, hkv, 128] bf16 (before the append)
    block_table: torch.Tensor      # [B, pages_per_row] int32, logical -> physical
    ctx_len: np.ndarray            # [B] tokens after the append
    q_len: np.ndarray              # [B]
    is_draft: np.ndarray           # [B] bool
    draft_pages: list              # per row: logical page ids (draft rows) or None
    q: torch.Tensor                # [T, hq, 128] bf16
    k_new: torch.Tensor            # [T, hkv, 128] bf16
    v_new: torch.Tensor            # [T, hkv, 128] bf16
    # mixed page list (the pages each row attends), reference layout with the
    # trailing padding row: qo/kv indptr [B+2], last_page_len [B+1]
    qo_indptr: torch.Tensor
    kv_indptr: torch.Tensor
    kv_indices: torch.Tensor
    last_page_len: torch.Tensor
    qo_indptr_host: torch.Tensor
    kv_indptr_host: torch.Tensor
    kv_len_host: torch.Tensor      # [B+1] tokens of each row's list (0 for padding)
    mode_flags: torch.Tensor       # [B] int32, 0 = draft
    extra: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return int(self.ctx_len.shape[0])

    @property
    def total_tokens(self) -> int:
        return int(self.q_len.sum())

    def list_pages(self) -> np.ndarray:
        return np.diff(self.kv_indptr_host.numpy()[: self.batch + 1])

    def algorithmic_bytes(self, include_append: bool = True) -> dict:
        """HBM bytes the layer must move: KV pages read, q + o, append, page ids."""
        kv = int(self.kv_len_host.numpy()[: self.batch].astype(np.int64).sum()) * self.hkv * HEAD_DIM * 2 * 2
        qo = self.total_tokens * self.hq * HEAD_DIM * 2 * 2
        app = self.total_tokens * self.hkv * HEAD_DIM * 2 * 2 * 2 if include_append else 0
        idx = int(self.list_pages().sum()) * 4
        return {"kv": kv, "qo": qo, "append": app, "indices": idx, "total": kv + qo + app + idx}


def _randn(shape, gen, device, dtype=torch.bfloat16, chunk=1 << 28):
    """N(0,1) on ``device`` generated in chunks (bounded temporaries)."""
    out = torch.empty(shape, dtype=dtype, device=device)
    flat = out.view(-1)
    for s in range(0, flat.numel(), chunk):
        e = min(s + chunk, flat.numel())
        flat[s:e] = torch.randn(e - s, generator=gen, device=device, dtype=torch.float32).to(dtype)
    return out


def build_step(*, hq: int, hkv: int, ctx_len, q_len, is_draft, draft_budget: int, pool_pages: int | None = None,
               seed: int = 0, device="cpu", key_bias_std: float = 0.5, draft_pages=None,
               bucket_tokens: int | None = None) -> MixedStep:
    """Build one mixed layer step. ``draft_pages`` (optional) gives each draft
    row's logical page selection; otherwise a seeded random subset of
    ``draft_budget - 1`` earlier pages plus the last page is used."""
    device = torch.device(device)
    ctx_len = np.asarray(ctx_len, dtype=np.int64)
    q_len = np.asarray(q_len, dtype=np.int64)
    is_draft = np.asarray(is_draft, dtype=bool)
    B = ctx_len.shape[0]
    rng = np.random.default_rng(seed)
    gen = torch.Generator(device=device).manual_seed(seed)
    pages_per_row = (ctx_len + PAGE - 1) // PAGE
    width = int(pages_per_row.max())
    total_pages = int(pages_per_row.sum())
    pool = pool_pages if pool_pages is not None else total_pages
    if pool < total_pages:
        raise ValueError("pool smaller than the pages the batch needs")
    perm = rng.permutation(pool).astype(np.int32)
    table = np.zeros((B, width), dtype=np.int32)
    off = 0
    for b in range(B):
        n = int(pages_per_row[b])
        table[b, :n] = perm[off : off + n]
        off += n

    cache = _randn((pool, 2, PAGE, hkv, HEAD_DIM), gen, device)
    if key_bias_std:
        bias = (torch.randn(pool, 1, hkv, 1, generator=gen, device=device) * key_bias_std)
        cache[:, 0] = (cache[:, 0].float() + bias).to(torch.bfloat16)

    T = int(q_len.sum())
    q = _randn((T, hq, HEAD_DIM), gen, device)
    k_new = _randn((T, hkv, HEAD_DIM), gen, device)
    v_new = _randn((T, hkv, HEAD_DIM), gen, device)

    sel = []
    lists = []
    for b in range(B):
        n = int(pages_per_row[b])
        if is_draft[b]:
            if draft_pages is not None and draft_pages[b] is not None:
                pages = np.asarray(sorted(draft_pages[b]), dtype=np.int64)
            else:
                k = min(draft_budget, n)
                pages = np.sort(np.concatenate([rng.choice(n - 1, size=k - 1, replace=False), [n - 1]])) \
                    if k > 1 else np.array([n - 1])
            sel.append(pages)
            lists.append(table[b, pages])
        else:
            sel.append(None)
            lists.append(table[b, :n])
    last = np.where(ctx_len > 0, (ctx_len - 1) % PAGE + 1, 0)
    list_pages = np.array([len(x) for x in lists], dtype=np.int64)
    kv_len = np.maximum(list_pages - 1, 0) * PAGE + last
    bucket = T if bucket_tokens is None else int(bucket_tokens)
    qo = np.zeros(B + 2, dtype=np.int32)
    qo[1 : B + 1] = np.cumsum(q_len)
    qo[B + 1] = bucket
    kvp = np.zeros(B + 2, dtype=np.int32)
    kvp[1 : B + 1] = np.cumsum(list_pages)
    kvp[B + 1] = kvp[B]
    lpl = np.zeros(B + 1, dtype=np.int32)
    lpl[:B] = last
    kvl = np.zeros(B + 1, dtype=np.int32)
    kvl[:B] = kv_len
    indices = np.concatenate(lists).astype(np.int32) if lists else np.zeros(0, np.int32)
    as_dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)
    return MixedStep(
        hq=hq, hkv=hkv, cache=cache, block_table=as_dev(table), ctx_len=ctx_len, q_len=q_len,
        is_draft=is_draft, draft_pages=sel, q=q, k_new=k_new, v_new=v_new,
        qo_indptr=as_dev(qo), kv_indptr=as_dev(kvp), kv_indices=as_dev(indices), last_page_len=as_dev(lpl),
        qo_indptr_host=torch.from_numpy(qo), kv_indptr_host=torch.from_numpy(kvp),
        kv_len_host=torch.from_numpy(kvl), mode_flags=as_dev(np.where(is_draft, 0, 1).astype(np.int32)),
    )


def config0(device="cpu", seed=0) -> MixedStep:
    """Qwen3-1.7B-shape layer, batch 4 x 4096 tokens (2 draft over 64 pages, 2 verify q_len 5)."""
    return build_step(hq=16, hkv=8, ctx_len=[4096] * 4, q_len=[1, 1, 5, 5], is_draft=[1, 1, 0, 0],
                      draft_budget=64, pool_pages=1024, seed=seed, device=device)


def config1(device="cpu", seed=0, batch: int = 32, ctx: int = 32768) -> MixedStep:
    """Qwen3-8B-shape layer, batch 32 x 32768 tokens (16 draft over 128 pages, 16 verify q_len 4)."""
    half = batch // 2
    return build_step(hq=32, hkv=8, ctx_len=[ctx] * batch, q_len=[1] * half + [4] * (batch - half),
                      is_draft=[1] * half + [0] * (batch - half), draft_budget=128,
                      pool_pages=batch * ((ctx + PAGE - 1) // PAGE), seed=seed, device=device)


def config2(device="cpu", seed=0, batch: int = 64, lo: int = 8192, hi: int = 32768) -> MixedStep:
    """Qwen3-8B refresh layer: batch 64, contexts U[8192, 32768], q_len 1, full attention."""
    rng = np.random.default_rng(seed + 1000)
    ctx = rng.integers(lo, hi + 1, size=batch)
    return build_step(hq=32, hkv=8, ctx_len=ctx, q_len=[1] * batch, is_draft=[0] * batch, draft_budget=0,
                      seed=seed, device=device)


def config4(device="cpu", seed=0, draft_frac: float = 0.0, batch: int = 16, lo: int = 65536,
            hi: int = 131072, draft_budget: int = 256) -> MixedStep:
    """Long-context layer: batch 16, contexts U[65536, 131072]; round(f * batch) seeded draft rows
    (q_len 1 over draft_budget pages), the others verify with q_len U{2..9}."""
    rng = np.random.default_rng(seed + 4000)
    ctx = rng.integers(lo, hi + 1, size=batch)
    n_draft = int(round(draft_frac * batch))
    is_draft = np.zeros(batch, dtype=bool)
    is_draft[rng.permutation(batch)[:n_draft]] = True
    q_len = np.where(is_draft, 1, rng.integers(2, 10, size=batch))
    return build_step(hq=32, hkv=8, ctx_len=ctx, q_len=q_len, is_draft=is_draft, draft_budget=draft_budget,
                      seed=seed, device=device)


def config3_rows(seed=0, batch: int = 64, lo: int = 8192, hi: int = 32768, draft_frac: float = 0.5,
                 q_lo: int = 2, q_hi: int = 9):
    """Rows of the full decode step: contexts U[lo, hi] (tokens after the append);
    round(draft_frac * batch) rows, chosen by a seeded permutation, draft (q_len 1)
    and the others verify with q_len U{q_lo..q_hi}. Returns (ctx_len, q_len, is_draft)."""
    rng = np.random.default_rng(seed + 3000)
    ctx = rng.integers(lo, hi + 1, size=batch).astype(np.int64)
    is_draft = np.zeros(batch, dtype=bool)
    is_draft[rng.permutation(batch)[: int(round(draft_frac * batch))]] = True
    q_len = np.where(is_draft, 1, rng.integers(q_lo, q_hi + 1, size=batch)).astype(np.int64)
    return ctx, q_len, is_draft


def random_block_table(pages_per_row, seed=0, pool_pages: int | None = None) -> tuple[np.ndarray, int]:
    """[B, max pages] int32 logical -> physical table drawn from a seeded
    permutation of the pool (default: exactly the pages the rows need)."""
    pages_per_row = np.asarray(pages_per_row, dtype=np.int64)
    total = int(pages_per_row.sum())
    pool = total if pool_pages is None else int(pool_pages)
    if pool < total:
        raise ValueError("pool smaller than the pages the rows need")
    perm = np.random.default_rng(seed + 77).permutation(pool).astype(np.int32)
    width = int(pages_per_row.max()) if pages_per_row.size else 0
    table = np.zeros((pages_per_row.size, width), dtype=np.int32)
    off = 0
    for b, n in enumerate(pages_per_row):
        table[b, :n] = perm[off : off + n]
        off += int(n)
    return table, pool
