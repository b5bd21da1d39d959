"""Host plan-array mirror: the CPU restatement pinned by hand-worked steps, and the
native HostPlanState (C++) against it over long random step sequences.

Reference: aspire/backends/host_plan.py (HostPlanConfig, HostPlanState.reset_all /
reset_slots / build_step)."""

import dataclasses

import numpy as np
import pytest

from aspire_amd.backends.host_plan import HostPlanConfig, HostPlanState
from oracle.host_plan import HostPlanMirror, last_page_len, num_pages, valid_count

BASE = dict(page_size=16, max_batch=4, draft_kind="gated", full_kind="effective_full", subset_cache_size=8,
            table_width=64, min_draft_pages=None, draft_percent=7.0, valid_floor_l=2, pages_per_slot=0)


def test_page_math_known_values():
    # the device helpers' documented examples (mixed_runner.py:98-120), page 128 and 16
    assert [last_page_len(n, 128) for n in (1, 128, 129, 0)] == [1, 128, 1, 0]
    assert [num_pages(n, 16) for n in (0, 1, 16, 17, 32768)] == [0, 1, 1, 2, 2048]


def test_percent_rule_rounds_in_fp32():
    cfg = dict(BASE, subset_cache_size=100, valid_floor_l=1)
    # 1500 * fp32(2.2) = 3300.0000715..., which rounds to 3300.0 in fp32: ceil(33.0) = 33
    # (in fp64 the product is 3300.0000000000005 and the ceil would be 34)
    assert valid_count(1500, dict(cfg, draft_percent=2.2)) == 33
    # floor and cap: 7% of 10 pages is 0.7 -> 1, raised to the floor 2; capped by the subset and by np
    assert valid_count(10, dict(cfg, valid_floor_l=2)) == 2
    assert valid_count(1000, dict(cfg, subset_cache_size=50)) == 50
    assert valid_count(1, cfg) == 1
    # explicit draft budget without a percentage: min(np, min_draft_pages)
    assert valid_count(40, dict(cfg, draft_percent=None, min_draft_pages=12)) == 12
    # sink_recent steps cap at the subset size, but its seeding follows the percent rule
    sr = dict(cfg, draft_kind="sink_recent", subset_cache_size=8, draft_percent=50.0)
    assert valid_count(10, sr) == 8 and valid_count(10, sr, seeding=True) == 5


def _step(m, **kw):
    return m.build_step(np.array(kw["verify"]), np.array(kw["finished"]), np.array(kw["draft_counts"]),
                        np.array(kw["seq_lens"]), kw["total_tokens"], kw["bucket_tokens"])


def test_gated_two_steps_by_hand():
    m = HostPlanMirror(BASE)
    m.reset_all([100, 200, 17, 5])
    assert m.draft_num_pages == [2, 2, 2, 1]
    # step 1: rows 0 and 3 verify (3 and 1 drafts), row 1 drafts, row 2 finished
    r = _step(m, verify=[1, 0, 0, 1], finished=[0, 0, 1, 0], draft_counts=[3, 2, 0, 1],
              seq_lens=[100, 200, 17, 5], total_tokens=7, bucket_tokens=8)
    assert r["dec"] == [4, 1, 0, 2]
    assert r["verify_num_pages"] == [7, 13, 2, 1] and r["effective_num_pages"] == [7, 13, 2, 1]
    assert r["last_page_len"] == [8, 11, 2, 7] and r["input_pos"] == [100, 202, 17, 5]
    assert r["qo_indptr"] == [0, 4, 5, 5, 7, 8]
    assert r["kv_indptr"] == [0, 7, 9, 11, 12, 12] and r["kv_len"] == [104, 27, 18, 7, 0]
    assert r["full_kv_indptr"] == [0, 7, 20, 22, 23, 23] and r["full_kv_len"] == [104, 203, 18, 7, 0]
    assert r["sample_indices"] == [0, 0, 0, 0, 1, 3, 3] and r["position_indices"] == [0, 1, 2, 3, 0, 0, 1]
    assert r["refresh_rows"] == [] and r["spill_rows"] == []
    # step 2: every row drafts; rows 0 and 3 verified last step (refreshed); row 1's draft
    # token is the first of a new page (206 + 2 + 1 = 209 = 13 * 16 + 1), so its table grows
    r = _step(m, verify=[0, 0, 0, 0], finished=[0, 0, 1, 0], draft_counts=[0, 2, 0, 0],
              seq_lens=[104, 206, 17, 7], total_tokens=3, bucket_tokens=4)
    assert r["refresh_rows"] == [0, 3] and r["spill_rows"] == [1]
    assert r["draft_num_pages"] == [2, 3, 2, 1]
    assert r["qo_indptr"] == [0, 1, 2, 2, 3, 4]
    assert r["kv_indptr"] == [0, 2, 5, 7, 8, 8] and r["kv_len"] == [25, 33, 18, 8, 0]
    assert r["input_pos"] == [104, 208, 17, 7]
    assert r["full_kv_indptr"] == [0, 7, 21, 23, 24, 24] and r["full_kv_len"] == [105, 209, 18, 8, 0]


def test_replan_mirror_and_static_full_layout_by_hand():
    m = HostPlanMirror(dict(BASE, draft_kind="replan", full_kind="mirror", draft_percent=None, min_draft_pages=5))
    m.reset_all([64, 64, 64, 64])
    r = _step(m, verify=[0, 1, 0, 1], finished=[0, 0, 0, 0], draft_counts=[1, 2, 0, 0],
              seq_lens=[95, 40, 3, 200], total_tokens=6, bucket_tokens=8)
    assert r["dec"] == [1, 3, 1, 1] and r["qo_indptr"] == [0, 1, 4, 5, 6, 8]
    # draft rows 0, 2: min(pages, 5) of the target length after the append (97 -> 7 pages, 4 -> 1 page)
    assert r["draft_num_pages"][:4] == [5, 3, 1, 5]   # replan refreshes every row (verify rows too)
    assert r["kv_indptr"] == [0, 5, 8, 9, 22, 22]       # verify rows: 43 -> 3 pages, 201 -> 13 pages
    assert r["kv_len"] == [64 + 1, 43, 4, 201, 0]        # draft row 0: 97 tokens, last page holds 1
    assert r["full_kv_indptr"] is r["kv_indptr"] and r["full_kv_len"] is r["kv_len"]
    s = HostPlanMirror(dict(BASE, draft_kind="sink_recent", pages_per_slot=10))
    s.reset_all([10, 10, 10, 10])
    r = _step(s, verify=[0, 0, 1, 0], finished=[0, 0, 0, 0], draft_counts=[0, 0, 0, 0],
              seq_lens=[10, 20, 30, 40], total_tokens=4, bucket_tokens=4)
    assert r["full_kv_indptr"] == [0, 10, 20, 30, 40, 40]
    assert r["full_kv_len"] == [11, 21, 31, 41, 0]


def test_token_total_mismatch_raises():
    m = HostPlanMirror(BASE)
    m.reset_all([10] * 4)
    with pytest.raises(RuntimeError):
        _step(m, verify=[0] * 4, finished=[0] * 4, draft_counts=[0] * 4, seq_lens=[10] * 4, total_tokens=5,
              bucket_tokens=8)
    h = HostPlanState(HostPlanConfig(**BASE))
    h.reset_all([10] * 4)
    with pytest.raises(RuntimeError):
        h.build_step(verify=np.zeros(4), finished=np.zeros(4), draft_counts=np.zeros(4, np.int64),
                     seq_lens=np.full(4, 10), total_tokens=5, bucket_tokens=8)


def _random_steps(cfg, steps, seed):
    rng = np.random.default_rng(seed)
    mb = cfg["max_batch"]
    seq = rng.integers(1, 4000, size=mb)
    return seq, [(rng.random(mb) < 0.5, rng.random(mb) < 0.1, rng.integers(0, 9, size=mb)) for _ in range(steps)]


CASES = [
    dict(BASE),
    dict(BASE, draft_kind="replan", full_kind=None, draft_percent=None, min_draft_pages=32),
    dict(BASE, draft_kind="sink_recent", full_kind="mirror", draft_percent=None),
    dict(BASE, draft_kind="gated", full_kind="effective_full", pages_per_slot=256, table_width=12),
    dict(BASE, draft_kind="gated", full_kind=None, draft_percent=2.2, subset_cache_size=64, max_batch=64),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_native_mirror_matches_oracle_over_steps(case):
    cfg = CASES[case]
    seq, steps = _random_steps(cfg, 60, seed=case)
    o = HostPlanMirror(cfg)
    n = HostPlanState(HostPlanConfig(**cfg))
    o.reset_all(seq)
    n.reset_all(seq)
    assert n.draft_num_pages.tolist() == o.draft_num_pages
    spills = refreshes = 0
    for i, (ver, fin, d) in enumerate(steps):
        d = np.where(ver, d, d % 3)
        dec = np.where(ver, d + 1, np.where(fin, 0, 1))
        tot = int(dec.sum())
        ro = o.build_step(ver, fin, d, seq, tot, tot + 3)
        rn = n.build_step(verify=ver, finished=fin, draft_counts=d, seq_lens=seq, total_tokens=tot,
                          bucket_tokens=tot + 3)
        for k in ("qo_indptr", "kv_indptr", "kv_len"):
            assert rn[k].tolist() == ro[k], (i, k)
        for k in ("dec", "verify_num_pages", "effective_num_pages", "last_page_len", "input_pos",
                  "sample_indices", "position_indices", "refresh_rows", "spill_rows", "draft_num_pages"):
            assert rn[k].tolist() == list(ro[k]), (i, k)
        if cfg["full_kind"] is None:
            assert rn["full_kv_indptr"] is None
        else:
            assert rn["full_kv_indptr"].tolist() == list(ro["full_kv_indptr"]), i
            assert rn["full_kv_len"].tolist() == list(ro["full_kv_len"]), i
        # invariants: the token split and the list lengths
        assert rn["qo_indptr"][len(seq)].item() == tot
        pages = np.diff(rn["kv_indptr"][: len(seq) + 1].numpy())
        kvl = rn["kv_len"][: len(seq)].numpy()
        assert np.all((kvl <= pages * 16) & ((pages == 0) | (kvl > (pages - 1) * 16)))
        spills += len(ro["spill_rows"])
        refreshes += len(ro["refresh_rows"])
        # next step: the caches grew by the accepted tokens
        seq = seq + np.where(ver, d + 1, 0)
    if cfg["draft_kind"] == "gated":  # both gated branches were exercised
        assert spills > 0 and refreshes > 0, (spills, refreshes)
    # slot refill
    o.reset_slots([1, 2], [5000, 7])
    n.reset_slots([1, 2], [5000, 7])
    assert n.draft_num_pages.tolist() == o.draft_num_pages


def test_native_config_round_trip():
    c = HostPlanConfig(**BASE)
    assert dataclasses.asdict(c)["draft_kind"] == "gated"
    with pytest.raises(ValueError):
        HostPlanState(dataclasses.replace(c, draft_kind="nope"))
