"""Host plan-array mirror, restated on the CPU (test infrastructure only).

Follows ``aspire/backends/host_plan.py``: the page math of ``_num_pages`` /
``_last_page_len`` (host_plan.py:84-90, the device's ``_get_num_pages`` /
``_get_last_page_len`` at aspire/models/mixed_runner.py:98-120), the draft
count rules ``_valid_counts`` / ``_init_counts`` (92-135, i.e.
``PageSelector.compute_valid_counts`` with its fp32 ceil, page_selector.py:52-62),
``reset_all`` / ``reset_slots`` (138-151) and ``build_step`` (155-306): per-row
decode tokens and cache lengths, the draft-table page counts of the three
refresh families, the spill / refresh rows, and the rendered plan arrays.

Written row by row in plain Python integers (the reference vectorises with
NumPy) so that it reads as an independent statement of the rules. One
deliberate difference: the reference's 'gated' branch combines a batch-sized
mask with a max_batch-sized one, which NumPy only accepts when the two sizes
are equal; this restatement uses the batch's rows, which is the same when they
are.

Pinned by: hand-worked known-answer steps (every refresh family, spill and
refresh rows, both full-context layouts, the percent rule's fp32 rounding) and
invariants in ``tests/test_host_plan_cpu.py``.
"""

from __future__ import annotations

import numpy as np

DRAFT_KINDS = ("replan", "sink_recent", "gated")
FULL_KINDS = (None, "mirror", "effective_full")


def num_pages(length: int, page: int) -> int:
    return (length + page - 1) // page


def last_page_len(length: int, page: int) -> int:
    return (length - 1) % page + 1 if length > 0 else 0


def valid_count(np_: int, cfg: dict, seeding: bool = False) -> int:
    """Draft pages a row keeps for ``np_`` target pages (host_plan.py:92-135)."""
    if cfg["draft_kind"] == "sink_recent" and not seeding:
        return min(np_, cfg["subset_cache_size"])
    hi = min(np_, cfg["subset_cache_size"])
    pct = cfg["draft_percent"]
    if pct is None:
        if cfg["min_draft_pages"] is not None:
            return min(np_, cfg["min_draft_pages"])
        return hi
    floor = cfg["min_draft_pages"] if cfg["min_draft_pages"] is not None else cfg["valid_floor_l"]
    lo = min(np_, floor)
    target = int(np.ceil(np.float32(np_) * np.float32(pct) / np.float32(100.0)))
    return min(max(target, lo), hi)


class HostPlanMirror:
    """State: draft page counts and last step's verify flags, max_batch rows each."""

    def __init__(self, cfg: dict):
        self.cfg = dict(cfg)
        self.draft_num_pages = [0] * cfg["max_batch"]
        self.prev_verify = [False] * cfg["max_batch"]

    def reset_all(self, seq_lens) -> None:
        for i, n in enumerate(seq_lens):
            self.draft_num_pages[i] = valid_count(num_pages(int(n), self.cfg["page_size"]), self.cfg, seeding=True)
        self.prev_verify = [False] * self.cfg["max_batch"]

    def reset_slots(self, slot_ids, seq_lens) -> None:
        for s, n in zip(slot_ids, seq_lens):
            self.draft_num_pages[int(s)] = valid_count(num_pages(int(n), self.cfg["page_size"]), self.cfg,
                                                       seeding=True)
            self.prev_verify[int(s)] = False

    def build_step(self, verify, finished, draft_counts, seq_lens, total_tokens: int, bucket_tokens: int) -> dict:
        cfg = self.cfg
        P = cfg["page_size"]
        mb = len(verify)
        out = {k: [] for k in ("dec", "verify_num_pages", "effective_num_pages", "last_page_len", "input_pos")}
        draft_cl = []
        for b in range(mb):
            ver = bool(verify[b])
            d = int(draft_counts[b])
            dec = d + 1 if ver else (0 if finished[b] else 1)
            cache = int(seq_lens[b]) + d - (d if ver else 0) + dec      # target cache after the append
            dcache = int(seq_lens[b]) + d + (0 if ver else 1)            # draft cache after the append
            eff = cache if ver else dcache
            out["dec"].append(dec)
            out["verify_num_pages"].append(num_pages(cache, P))
            out["effective_num_pages"].append(num_pages(eff, P))
            out["last_page_len"].append(last_page_len(eff, P))
            out["input_pos"].append(cache - dec if ver else dcache - 1)
            draft_cl.append(dcache)

        refresh, spill = [], []
        if cfg["draft_kind"] in ("replan", "sink_recent"):
            for b in range(mb):
                self.draft_num_pages[b] = valid_count(out["verify_num_pages"][b], cfg)
        else:
            refresh = [b for b in range(cfg["max_batch"]) if self.prev_verify[b]]
            for b in refresh:
                if b >= mb:
                    raise IndexError(f"row {b} verified last step but the batch is {mb} rows")
                self.draft_num_pages[b] = valid_count(out["verify_num_pages"][b], cfg)
            for b in range(mb):
                opens_page = (not verify[b]) and out["dec"][b] > 0 and (draft_cl[b] - 1) % P == 0
                if opens_page and not self.prev_verify[b] and self.draft_num_pages[b] < cfg["table_width"]:
                    self.draft_num_pages[b] += 1
                    spill.append(b)

        nq, nl = cfg["max_batch"] + 2, cfg["max_batch"] + 1
        qo, kvp, kvl = [0] * nq, [0] * nq, [0] * nl
        for b in range(mb):
            pages = out["verify_num_pages"][b] if verify[b] else self.draft_num_pages[b]
            qo[b + 1] = qo[b] + out["dec"][b]
            kvp[b + 1] = kvp[b] + pages
            kvl[b] = max(pages - 1, 0) * P + out["last_page_len"][b]
        for i in range(mb + 1, nq):
            qo[i] = bucket_tokens
            kvp[i] = kvp[mb]
        if qo[mb] != total_tokens:
            raise RuntimeError(f"host plan mirror diverged: token total {qo[mb]} != scheduler total {total_tokens}")

        sample, position = [], []
        for b in range(mb):
            sample += [b] * out["dec"][b]
            position += list(range(out["dec"][b]))

        res = {"qo_indptr": qo, "kv_indptr": kvp, "kv_len": kvl, "refresh_rows": refresh, "spill_rows": spill,
               "draft_num_pages": list(self.draft_num_pages), "sample_indices": sample,
               "position_indices": position, **out, "full_kv_indptr": None, "full_kv_len": None}
        if cfg["full_kind"] == "mirror":
            res["full_kv_indptr"], res["full_kv_len"] = kvp, kvl
        elif cfg["full_kind"] == "effective_full":
            fkvp, fkvl = [0] * nq, [0] * nl
            pps = cfg.get("pages_per_slot", 0)
            for b in range(mb):
                ep = out["effective_num_pages"][b]
                fkvp[b + 1] = (b + 1) * pps if pps > 0 else fkvp[b] + ep
                fkvl[b] = max(ep - 1, 0) * P + out["last_page_len"][b]
            for i in range(mb + 1, nq):
                fkvp[i] = fkvp[mb]
            res["full_kv_indptr"], res["full_kv_len"] = fkvp, fkvl
        for b in range(mb):
            self.prev_verify[b] = bool(verify[b])
        return res
