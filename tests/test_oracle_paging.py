"""Pins the oracle's page-table helpers (``page_table``, ``expand_pages``):
AITER's paged-cache arguments (mixed-mla/asm_dumps/aiter_mla.py:149-175) as
mixed-mla/submission.py:449-456 and :538-544 build them, expanded back to
token rows.  Pins: a round trip through a random page placement returns every
token's row; page_size 1 is the identity; ragged and empty sequences."""
import numpy as np
import pytest

from oracle import mla_oracle as O


@pytest.mark.parametrize("P", [1, 2, 8, 16, 64])
def test_round_trip_through_random_pages(P):
    rng = np.random.default_rng(P)
    lens = [0, 1, P, P + 1, 3 * P - 1, 1000, 0, 37]
    npages = [(L + P - 1) // P for L in lens]
    total = sum(npages)
    perm = rng.permutation(total + 11)  # spare pages stay unused
    cursor = [0]

    def ids_for(b, n):
        out = perm[cursor[0]:cursor[0] + n]
        cursor[0] += n
        return out

    indptr, ids, last = O.page_table(lens, P, ids_for)
    assert indptr[-1] == total and len(ids) == total
    assert np.all((last >= 1) & (last <= P))
    kv_indptr, kv_indices = O.expand_pages(indptr, ids, last, P)
    assert np.array_equal(np.diff(kv_indptr), lens)
    # token j of sequence b sits at offset j % P of its (j // P)-th page
    for b, L in enumerate(lens):
        rows = kv_indices[kv_indptr[b]:kv_indptr[b + 1]]
        j = np.arange(L)
        assert np.array_equal(rows, ids[indptr[b] + j // P] * P + j % P)
    assert len(np.unique(kv_indices)) == len(kv_indices)  # distinct pages -> distinct rows


def test_page_size_one_is_identity():
    lens = [5, 0, 9]
    idx = np.arange(14, dtype=np.int32)[::-1].copy()
    indptr, ids, last = O.page_table(lens, 1, lambda b, n: idx[[0, 5, 5][b]:[0, 5, 5][b] + n])
    kv_indptr, kv_indices = O.expand_pages(indptr, ids, last, 1)
    assert np.array_equal(kv_indptr, [0, 5, 5, 14])
    assert np.array_equal(kv_indices, idx)


def test_last_page_length_is_clamped():
    # a last_page_lens entry above P counts as P, below 1 as 1
    indptr = np.array([0, 2, 3], np.int32)
    ids = np.array([4, 1, 7], np.int32)
    kv_indptr, kv_indices = O.expand_pages(indptr, ids, np.array([9, 0], np.int32), 4)
    assert np.array_equal(kv_indptr, [0, 8, 9])
    assert np.array_equal(kv_indices, [16, 17, 18, 19, 4, 5, 6, 7, 28])
