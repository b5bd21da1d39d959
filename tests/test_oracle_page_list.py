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
