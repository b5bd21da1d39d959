"""The CPU append oracle: a hand-worked case and invariants."""

import numpy as np

from oracle.append import batch_indices_positions, paged_kv_append, seq_lens


def test_hand_worked_case():
    # page 4, 2 rows. Row 0 owns pages [5, 2] with last_page_len 3 -> kv_len 7;
    # row 1 owns page [0] with last_page_len 2 -> kv_len 2. Append 2 tokens to
    # row 0 and 1 to row 1; token 3 is bucket padding.
    kv_indptr = np.array([0, 2, 3, 3])
    last = np.array([3, 2, 0])
    assert seq_lens(kv_indptr, last, 4).tolist() == [7, 2, 0]
    append_indptr = np.array([0, 2, 3, 4])
    b, p = batch_indices_positions(append_indptr, seq_lens(kv_indptr, last, 4), 4)
    assert b.tolist() == [0, 0, 1, 2] and p.tolist() == [5, 6, 1, -1]
    H, D = 1, 2
    k = np.arange(4 * H * D, dtype=np.uint16).reshape(4, H, D) + 100
    v = k + 1000
    cache = np.zeros((6, 2, 4, H, D), dtype=np.uint16)
    out = paged_kv_append(k, v, append_indptr, cache, np.array([5, 2, 0]), kv_indptr, last, 4)
    # token 0 -> pos 5 -> logical page 1 (phys 2), slot 1; token 1 -> pos 6 -> phys 2 slot 2
    assert (out[2, 0, 1, 0] == k[0, 0]).all() and (out[2, 1, 1, 0] == v[0, 0]).all()
    assert (out[2, 0, 2, 0] == k[1, 0]).all() and (out[2, 1, 2, 0] == v[1, 0]).all()
    # token 2 -> row 1 pos 1 -> phys 0 slot 1
    assert (out[0, 0, 1, 0] == k[2, 0]).all()
    # nothing else changed
    touched = np.zeros_like(out, dtype=bool)
    touched[2, :, 1] = touched[2, :, 2] = touched[0, :, 1] = True
    assert (out[~touched] == 0).all()


def test_roundtrip_and_untouched_bytes():
    rng = np.random.default_rng(0)
    page, H, D, P = 16, 3, 8, 64
    lens = np.array([37, 16, 1, 50])
    qlens = np.array([1, 4, 1, 3])
    npages = (lens + page - 1) // page
    kv_indptr = np.concatenate([[0], np.cumsum(npages), [npages.sum()]])
    kv_indices = rng.permutation(P)[: npages.sum()]
    last = np.concatenate([(lens - 1) % page + 1, [0]])
    append_indptr = np.concatenate([[0], np.cumsum(qlens)])
    T = int(append_indptr[-1]) + 2  # two bucket-padding tokens
    append_indptr = np.concatenate([append_indptr, [T]])
    k = rng.integers(0, 65535, size=(T, H, D), dtype=np.uint16)
    v = rng.integers(0, 65535, size=(T, H, D), dtype=np.uint16)
    cache = rng.integers(0, 65535, size=(P, 2, page, H, D), dtype=np.uint16)
    out = paged_kv_append(k, v, append_indptr, cache, kv_indices, kv_indptr, last, page)
    written = np.zeros(out.shape[:3], dtype=bool)
    for b in range(4):
        for n in range(qlens[b]):
            pos = lens[b] - qlens[b] + n
            phys = kv_indices[kv_indptr[b] + pos // page]
            tok = append_indptr[b] + n
            assert (out[phys, 0, pos % page] == k[tok]).all()
            assert (out[phys, 1, pos % page] == v[tok]).all()
            written[phys, :, pos % page] = True
    assert (out[~written] == cache[~written]).all()
