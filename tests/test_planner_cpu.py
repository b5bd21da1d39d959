"""Host planner invariants (pure host code in libaspire_hip.so; no GPU needed)."""

import ctypes
from pathlib import Path

import numpy as np
import pytest
import torch

from aspire_amd import _lib

LIB = Path(_lib.LIB_PATH)
pytestmark = pytest.mark.skipif(not LIB.exists(), reason="libaspire_hip.so not built")

HEADER_INTS = 32


def layout(num_cus=256, waves_per_cu=8, float_ws=384 << 20):
    lay = _lib.PlanLayout()
    rc = _lib.lib().aspire_plan_layout_init(num_cus, waves_per_cu, 8 << 20, float_ws, 128, ctypes.byref(lay))
    _lib.check(rc, "layout")
    return lay


def offsets(lay):
    W = lay.num_waves
    cur = HEADER_INTS
    indptr = []
    for _ in range(3):
        indptr.append(cur)
        cur += W + 1
    cur = (cur + 7) & ~7
    items = []
    for _ in range(3):
        items.append(cur)
        cur += lay.max_items * 8
    return indptr, items, cur


def plan(lay, qo, kvp, kvl, hq, hkv, per_head=False, causal=True):
    buf = np.zeros(8 << 18, dtype=np.int32)
    info = _lib.PlanInfo()
    qo = np.ascontiguousarray(qo, dtype=np.int32)
    kvp = np.ascontiguousarray(kvp, dtype=np.int32)
    kvl = np.ascontiguousarray(kvl, dtype=np.int32)
    batch = len(kvl) // hkv if per_head else len(kvl)
    rc = _lib.lib().aspire_plan_build(
        ctypes.byref(lay), qo.ctypes.data_as(ctypes.c_void_p), kvp.ctypes.data_as(ctypes.c_void_p),
        kvl.ctypes.data_as(ctypes.c_void_p), batch, int(per_head), hq, hkv, 16, int(causal),
        buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes, ctypes.byref(info))
    _lib.check(rc, "plan")
    return buf, info


def decode(lay, buf, info):
    indptr_off, items_off, merge_off = offsets(lay)
    W = lay.num_waves
    classes = []
    for c in range(3):
        ip = buf[indptr_off[c] : indptr_off[c] + W + 1]
        it = buf[items_off[c] : items_off[c] + info.num_items[c] * 8].reshape(-1, 8)
        classes.append((ip, it))
    merges = buf[merge_off : merge_off + info.num_merge * 8].reshape(-1, 8)
    return classes, merges


def expected_tiles(q_len, kv_len, group, causal=True):
    """Query tiles of a row, (t0, tq, keys): rows longer than 48 query rows are cut into
    tiles of 48 // group tokens whose keys end at their last token (causal)."""
    tile = max(1, 48 // group)
    if q_len * group <= 48:
        return [(0, q_len, kv_len)]
    return [(t0, min(tile, q_len - t0), max(kv_len - q_len + t0 + min(tile, q_len - t0), 0) if causal else kv_len)
            for t0 in range(0, q_len, tile)]


DIRECT = 1 << 16  # item flag: heads of a head-aligned row read different lists


def check_cover(lay, buf, info, qo, kvp, kvl, hq, hkv, per_head=False, causal=True, seg_start=None):
    classes, merges = decode(lay, buf, info)
    group = hq // hkv
    hpu = int(buf[4])
    starts = np.asarray(seg_start) if seg_start is not None else np.asarray(kvp)[: len(kvl)]
    seen = {}
    partial_rows = set()
    for c, (ip, it) in enumerate(classes):
        assert ip[0] == 0 and ip[-1] == len(it) and np.all(np.diff(ip) >= 0)
        for w in range(lay.num_waves):
            for row in it[ip[w] : ip[w + 1]]:
                q_start, q_len, kv_len, base, pb, pe, bg, prow = row.tolist()
                flag, q_len = q_len & DIRECT, q_len & (DIRECT - 1)
                b, g = bg >> 8, bg & 255
                shared = not per_head or len(set(starts[b * hkv : (b + 1) * hkv].tolist())) == 1
                assert bool(flag) == (hpu > 1 and not shared), (b, g, flag, hpu)
                assert (q_len * group - 1) // 16 == c
                seg = b * hkv + g if per_head else b
                tiles = {t0: (tq, keys) for t0, tq, keys in
                         expected_tiles(qo[b + 1] - qo[b], kvl[seg], group, causal)}
                t0 = q_start - qo[b]
                assert t0 in tiles and (q_len, kv_len) == tiles[t0], (b, t0, q_len, kv_len)
                assert base == starts[seg] and pe <= (kv_len + 15) // 16
                for p in range(pb, pe):
                    key = (b, g, t0, p)
                    assert key not in seen, f"page {key} planned twice"
                    seen[key] = prow
                if prow >= 0:
                    for r in range(q_len * group):
                        assert prow + r not in partial_rows
                        partial_rows.add(prow + r)
    # every page of every query tile of every segment with queries is covered exactly once
    nrows = len(kvl) // hkv if per_head else len(kvl)
    for b in range(min(len(qo) - 1, nrows)):
        if qo[b + 1] - qo[b] <= 0:
            continue
        for g in range(hkv):
            seg = b * hkv + g if per_head else b
            for t0, tq, keys in expected_tiles(qo[b + 1] - qo[b], kvl[seg], group, causal):
                for p in range((keys + 15) // 16):
                    assert (b, g, t0, p) in seen
    # merge items reference the split pieces; their row ranges cover each split segment's rows
    # once, in ranges the merge kernel's piece groups fit (48 rows, or 24 / 12 rows for items of
    # more than 8 / 16 pieces)
    covered = {}
    for m in merges:
        q_start, q_len, bg, first, pieces, rows, row_begin, row_count = m.tolist()
        assert pieces >= 2 and rows == q_len * group
        assert 0 <= row_begin and 0 < row_count and row_begin + row_count <= rows
        assert row_count <= (12 if pieces > 16 else 24 if pieces > 8 else 48)
        for k in range(pieces):
            assert first + k * rows in partial_rows
        got = covered.setdefault((q_start, bg, first), set())
        assert got.isdisjoint(range(row_begin, row_begin + row_count))
        got.update(range(row_begin, row_begin + row_count))
    for (q_start, bg, first), got in covered.items():
        q_len = next(int(m[1]) for m in merges if (m[0], m[2], m[3]) == (q_start, bg, first))
        assert got == set(range(q_len * group))
    return seen


def test_cover_and_balance_config1_shape():
    B, hq, hkv = 32, 32, 8
    q_len = np.array([1] * 16 + [4] * 16)
    kvl = np.array([128 * 16] * 16 + [32768] * 16 + [0])
    pages = (kvl + 15) // 16
    qo = np.concatenate([[0], np.cumsum(q_len), [80]])
    kvp = np.concatenate([[0], np.cumsum(pages[:B]), [pages[:B].sum()]])
    lay = layout()
    buf, info = plan(lay, qo, kvp, kvl, hq, hkv)
    check_cover(lay, buf, info, qo, kvp, kvl, hq, hkv)
    assert info.total_pages == int(pages[:B].sum()) * hkv
    # stream-K balance: every wave streams floor or ceil of the mean page count
    classes, _ = decode(lay, buf, info)
    ip, it = classes[0]
    per_wave = np.array([int((it[ip[w]:ip[w + 1], 5] - it[ip[w]:ip[w + 1], 4]).sum()) for w in range(lay.num_waves)])
    mean = info.total_pages / lay.num_waves
    assert per_wave.max() <= np.ceil(mean) and per_wave.min() >= np.floor(mean)


def test_mixed_classes_ragged_and_empty_rows():
    hq, hkv = 32, 8
    q_len = np.array([1, 2, 5, 9, 0, 3, 12 // 4 * 4 // 4, 1])
    kvl = np.array([37, 0, 4096 + 5, 100000, 50, 17, 16, 1, 0])
    pages = (kvl + 15) // 16
    B = len(q_len)
    qo = np.concatenate([[0], np.cumsum(q_len), [q_len.sum() + 3]])
    kvp = np.concatenate([[0], np.cumsum(pages[:B]), [pages[:B].sum()]])
    kvl_full = np.concatenate([kvl[:B], [0]])
    lay = layout(num_cus=16, waves_per_cu=4)
    buf, info = plan(lay, qo, kvp, kvl_full, hq, hkv)
    check_cover(lay, buf, info, qo, kvp, kvl_full, hq, hkv)
    assert info.num_items[2] > 0 and info.num_merge > 0


def test_per_head_lists():
    hq, hkv, B = 32, 8, 3
    rng = np.random.default_rng(0)
    kvl = rng.integers(1, 3000, size=B * hkv)
    pages = (kvl + 15) // 16
    kvp = np.concatenate([[0], np.cumsum(pages)])
    qo = np.array([0, 1, 2, 3])
    lay = layout(num_cus=8, waves_per_cu=4)
    buf, info = plan(lay, qo, kvp, kvl, hq, hkv, per_head=True)
    assert int(buf[4]) == 1  # heads of a row differ in length: one wave per (row, head)
    check_cover(lay, buf, info, qo, kvp, kvl, hq, hkv, per_head=True)
    # one length per row: head-aligned slots, every row's heads on their own lists (flagged)
    kvl_u = np.repeat(kvl[::hkv], hkv)
    kvp_u = np.concatenate([[0], np.cumsum((kvl_u + 15) // 16)])
    buf, info = plan(lay, qo, kvp_u, kvl_u, hq, hkv, per_head=True)
    assert int(buf[4]) == hkv
    check_cover(lay, buf, info, qo, kvp_u, kvl_u, hq, hkv, per_head=True)


def test_rejects_bad_inputs():
    lay = layout(num_cus=4, waves_per_cu=4)
    with pytest.raises(ValueError, match="pages"):
        plan(lay, np.array([0, 1]), np.array([0, 1]), np.array([40]), 32, 8)  # list shorter than kv_len
    with pytest.raises(ValueError, match="multiple"):
        plan(lay, np.array([0, 1]), np.array([0, 1]), np.array([16]), 30, 8)


def test_partial_capacity_shrinks_split():
    hq, hkv = 32, 8
    kvl = np.array([32768] * 4 + [0])
    qo = np.array([0, 4, 8, 12, 16, 16])
    pages = (kvl + 15) // 16
    kvp = np.concatenate([[0], np.cumsum(pages[:4]), [pages[:4].sum()]])
    small = layout(num_cus=64, waves_per_cu=8, float_ws=40 * 129 * 4 * 16)
    buf, info = plan(small, qo, kvp, kvl, hq, hkv)
    assert info.partial_rows <= small.partial_rows_cap
    check_cover(small, buf, info, qo, kvp, kvl, hq, hkv)


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_rows_split_into_query_tiles(causal):
    """Chunked prefill: rows of 300 and 1000 new tokens over prefixes of 700 and 0 tokens (GQA 4:
    tiles of 12 tokens), beside a decode row."""
    hq, hkv = 32, 8
    qo = np.array([0, 300, 1300, 1301])
    kvl = np.array([1000, 1000, 5000])
    pages = (kvl + 15) // 16
    kvp = np.concatenate([[0], np.cumsum(pages)])
    lay = layout(num_cus=16, waves_per_cu=4)
    buf, info = plan(lay, qo, kvp, kvl, hq, hkv, causal=causal)
    assert info.split_rows == 2 and info.max_rows == 48
    check_cover(lay, buf, info, qo, kvp, kvl, hq, hkv, causal=causal)
    # the first tile of the second row only needs the keys up to its 12th token
    if causal:
        assert expected_tiles(1000, 1000, 4)[0] == (0, 12, 12)


def plan_segments(lay, qo, start, pages, kvl, hq, hkv, causal=True):
    buf = np.zeros(8 << 18, dtype=np.int32)
    info = _lib.PlanInfo()
    arr = lambda a: np.ascontiguousarray(a, dtype=np.int32)
    qo, start, pages, kvl = arr(qo), arr(start), arr(pages), arr(kvl)
    rc = _lib.lib().aspire_plan_build_segments(
        ctypes.byref(lay), qo.ctypes.data_as(ctypes.c_void_p), start.ctypes.data_as(ctypes.c_void_p),
        pages.ctypes.data_as(ctypes.c_void_p), kvl.ctypes.data_as(ctypes.c_void_p), len(kvl) // hkv, hq, hkv, 16,
        int(causal), buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes, ctypes.byref(info))
    _lib.check(rc, "plan_segments")
    return buf, info


def test_segments_shared_and_per_head_rows():
    """Verify rows share one list across heads (staged), draft rows hold one per head (flagged
    direct); all heads of a row have one length, so the plan is head-aligned."""
    hq, hkv = 32, 8
    rng = np.random.default_rng(2)
    ctx = np.array([5000, 700, 3000, 123, 64, 2000])
    ql = np.array([1, 4, 1, 9, 1, 2])
    draft = ql == 1
    cnt = np.where(draft, np.minimum(40, (ctx + 15) // 16), (ctx + 15) // 16)
    start = np.zeros((len(ctx), hkv), dtype=np.int64)
    pos = 0
    for b in range(len(ctx)):
        if draft[b]:
            start[b] = pos + cnt[b] * np.arange(hkv)
            pos += cnt[b] * hkv
        else:
            start[b] = pos
            pos += cnt[b]
    start = start.reshape(-1)
    pages = np.repeat(cnt, hkv)
    kvl = np.repeat((cnt - 1) * 16 + (ctx - 1) % 16 + 1, hkv)
    qo = np.concatenate([[0], np.cumsum(ql)])
    lay = layout(num_cus=16, waves_per_cu=4)
    buf, info = plan_segments(lay, qo, start, pages, kvl, hq, hkv)
    assert int(buf[4]) == hkv
    check_cover(lay, buf, info, qo, None, kvl, hq, hkv, per_head=True, seg_start=start)
    # one head of one row longer than its siblings: per-(row, head) slots, no flags
    kvl2 = kvl.copy()
    kvl2[3] -= 16
    buf2, info2 = plan_segments(lay, qo, start, pages, kvl2, hq, hkv)
    assert int(buf2[4]) == 1
    check_cover(lay, buf2, info2, qo, None, kvl2, hq, hkv, per_head=True, seg_start=start)
    # a list shorter than its length is rejected
    with pytest.raises(ValueError, match="pages"):
        bad = pages.copy()
        bad[5] -= 1
        plan_segments(lay, qo, start, bad, kvl, hq, hkv)


def test_rejects_gqa_group_wider_than_three_tiles():
    """A query token's GQA group must fit one 3-tile item (48 rows): 64 q heads over one
    kv head is refused with ASPIRE_ERR_INVALID instead of planned past the last class."""
    lay = layout(num_cus=16, waves_per_cu=4)
    qo = np.array([0, 1], dtype=np.int32)
    kvp = np.array([0, 4], dtype=np.int32)
    kvl = np.array([64], dtype=np.int32)
    buf = np.zeros(8 << 18, dtype=np.int32)
    info = _lib.PlanInfo()
    rc = _lib.lib().aspire_plan_build(
        ctypes.byref(lay), qo.ctypes.data_as(ctypes.c_void_p), kvp.ctypes.data_as(ctypes.c_void_p),
        kvl.ctypes.data_as(ctypes.c_void_p), 1, 0, 64, 1, 16, 1, buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes,
        ctypes.byref(info))
    assert rc == _lib.ASPIRE_ERR_INVALID
    assert "at most 48" in _lib.lib().aspire_last_error().decode()
    # the widest accepted group (48 q heads per kv head) still plans
    plan(lay, qo, kvp, kvl, 48, 1)


def test_config3_layer_cost_balance():
    """A config-3 mixed layer (64 rows, contexts U[8k, 32k], per-head top-128 draft lists, verify
    q_len U{2..9}) on 256 CUs: the three row-tile classes form one stream-K sequence in cost
    units (quarters: 33 per staged 1-tile page, 32 per staged 2-/3-tile page, 48 per per-head
    page), so every slot streams the mean cost to within one page, and no merge needs more than
    one round of loads."""
    from aspire_amd.workloads import PAGE, config3_rows

    ctx, ql, dr = config3_rows(seed=0)
    hq, hkv = 32, 8
    starts, pages, kvl = [], [], []
    pos = 0
    for b in range(len(ctx)):
        n = (int(ctx[b]) + PAGE - 1) // PAGE
        for g in range(hkv):
            starts.append(pos + g * 128 if dr[b] else pos)
            pages.append(128 if dr[b] else n)
            kvl.append(127 * PAGE + int(ctx[b]) - (n - 1) * PAGE if dr[b] else int(ctx[b]))
        pos += 128 * hkv if dr[b] else n
    qo = np.concatenate([[0], np.cumsum(ql)])
    lay = layout(num_cus=256, waves_per_cu=4)
    buf, info = plan_segments(lay, qo, starts, pages, kvl, hq, hkv)
    check_cover(lay, buf, info, qo, None, np.array(kvl), hq, hkv, per_head=True, seg_start=np.array(starts))
    classes, merges = decode(lay, buf, info)
    hpu = int(buf[4])
    assert hpu == hkv
    cost = np.zeros(lay.num_waves)
    for c, (ip, it) in enumerate(classes):
        for w in range(lay.num_waves):
            for row in it[ip[w] : ip[w + 1]]:
                direct = (int(row[1]) & DIRECT) != 0
                cost[w] += (int(row[5]) - int(row[4])) * (48 if direct else 33 if c == 0 else 32)
    slot_cost = cost[::hpu]
    assert slot_cost.max() - slot_cost.min() <= 2 * 48
    assert (merges[:, 4] <= 8).all()


def test_merge_row_ranges_lone_long_row():
    """One 131,072-token verify row with q_len 9 at GQA 4 (36 rows, 3 tiles) beside a short draft
    row: the long row streams over every slot, and its 36-row merges come as row ranges of 12 rows,
    so that four lane groups share each row's pieces."""
    hq, hkv = 32, 8
    ql = np.array([9, 1])
    kvl = np.array([131072, 300])
    pages = (kvl + 15) // 16
    qo = np.concatenate([[0], np.cumsum(ql)])
    kvp = np.concatenate([[0], np.cumsum(pages)])
    lay = layout(num_cus=256, waves_per_cu=4)
    buf, info = plan(lay, qo, kvp, kvl, hq, hkv)
    check_cover(lay, buf, info, qo, kvp, kvl, hq, hkv)
    _, merges = decode(lay, buf, info)
    long = merges[merges[:, 5] == 36]
    assert len(long) and (long[:, 4] > 16).all() and (long[:, 7] == 12).all()
