"""The CPU page-list oracle: a hand-worked case."""

import numpy as np

from oracle.page_list import build_unified_indices, fill_padding_rows


def test_hand_worked_case():
    mode = np.array([0, 1, 0, 1])
    draft = np.array([[9, 8, 7], [1, 1, 1], [4, 5, 6], [2, 2, 2]])
    verify = np.array([[10, 11, 12, 13], [20, 21, 22, 23], [30, 31, 32, 33], [40, 41, 42, 43]])
    dn = np.array([2, 3, 3, 1])
    vn = np.array([4, 1, 4, 3])
    idx = np.full(20, -7)
    indptr = np.full(7, -1)
    build_unified_indices(mode, draft, verify, dn, vn, idx, indptr)
    assert indptr[:5].tolist() == [0, 2, 3, 6, 9]
    assert idx[:9].tolist() == [9, 8, 20, 4, 5, 6, 40, 41, 42]
    assert (idx[9:] == -7).all()
    last = np.array([5, 6, 7, 8, 9, 9])
    fill_padding_rows(indptr, last, 4)
    assert indptr.tolist() == [0, 2, 3, 6, 9, 9, 9] and last.tolist() == [5, 6, 7, 8, 0, 0]


def test_head_lists_hand_worked_case():
    from oracle.page_list import build_head_page_lists
    mode = np.array([1, 0])
    sel = np.array([[[0, 0, 0], [0, 0, 0]], [[7, 9, 0], [3, 0, 0]]])
    cnt = np.array([[0, 0], [2, 1]])
    table = np.array([[10, 11, 12], [20, 21, 22]])
    vn = np.array([2, 3])
    idx = np.full(12, -1)
    ptr = np.full(5, -1)
    build_head_page_lists(mode, sel, cnt, table, vn, idx, ptr)
    assert ptr.tolist() == [0, 2, 4, 6, 7]
    assert idx[:7].tolist() == [10, 11, 10, 11, 7, 9, 3] and (idx[7:] == -1).all()


def test_head_lists_reduce_to_row_lists():
    """With every head holding the row's selection, each segment is the row list of the
    pinned per-row builder; with one head the two builders agree entry for entry."""
    from oracle.page_list import build_head_page_lists
    rng = np.random.default_rng(3)
    B, H, W, K = 6, 4, 40, 12
    mode = rng.integers(0, 2, B)
    table = rng.integers(0, 10000, (B, W))
    dn = rng.integers(0, K + 1, B)
    vn = rng.integers(0, W + 1, B)
    draft = rng.integers(0, 10000, (B, K))
    row_idx = np.zeros(B * W, dtype=np.int64)
    row_ptr = np.zeros(B + 1, dtype=np.int64)
    build_unified_indices(mode, draft, table, dn, vn, row_idx, row_ptr)
    sel = np.repeat(draft[:, None, :], H, axis=1)
    cnt = np.repeat(dn[:, None], H, axis=1)
    idx = np.zeros(B * H * W, dtype=np.int64)
    ptr = np.zeros(B * H + 1, dtype=np.int64)
    build_head_page_lists(mode, sel, cnt, table, vn, idx, ptr)
    for b in range(B):
        row = row_idx[row_ptr[b] : row_ptr[b + 1]]
        for g in range(H):
            s = b * H + g
            assert np.array_equal(idx[ptr[s] : ptr[s + 1]], row)
    idx1 = np.zeros(B * W, dtype=np.int64)
    ptr1 = np.zeros(B + 1, dtype=np.int64)
    build_head_page_lists(mode, draft[:, None, :], dn[:, None], table, vn, idx1, ptr1)
    assert np.array_equal(ptr1, row_ptr) and np.array_equal(idx1[: ptr1[-1]], row_idx[: row_ptr[-1]])


def test_head_lists_shared_verify_rows():
    """With sharing, a verify row's heads all start at one copy of its table and the
    draft rows' lists are the unshared ones, shifted."""
    from oracle.page_list import build_head_page_lists
    mode = np.array([0, 1, 0])
    H = 3
    sel = np.arange(3 * H * 4).reshape(3, H, 4) + 100
    cnt = np.array([[2, 1, 3], [0, 0, 0], [1, 1, 1]])
    table = np.array([[1, 2, 3, 4], [5, 6, 7, 8], [9, 10, 11, 12]])
    vn = np.array([4, 3, 4])
    idx = np.full(30, -1)
    ptr = np.full(3 * H + 1, -1)
    build_head_page_lists(mode, sel, cnt, table, vn, idx, ptr, share_verify=True)
    assert ptr.tolist() == [0, 2, 3, 6, 6, 6, 9, 10, 11, 12]
    assert idx[:12].tolist() == [100, 101, 104, 108, 109, 110, 5, 6, 7, 124, 128, 132]
    assert (idx[12:] == -1).all()
