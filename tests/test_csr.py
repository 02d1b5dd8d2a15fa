"""CSR page-list adapter: reference competitors.py:8-18 semantics and its inverse."""
import numpy as np
import pytest

from paged_decode.csr import from_csr, paged_csr
from paged_decode.layout import Layout
from paged_decode.workload import make_metadata


def test_known_answer():
    layout = Layout(3, 4, 2, 64, 16, 10)
    table = np.array([[3, 1, -1], [0, 2, 4], [9, -1, -1]], dtype=np.int32)
    lengths = np.array([17, 48, 5], dtype=np.int32)
    indptr, indices, last = paged_csr(layout, table, lengths)
    np.testing.assert_array_equal(indptr, [0, 2, 5, 6])
    np.testing.assert_array_equal(indices, [3, 1, 0, 2, 4, 9])
    np.testing.assert_array_equal(last, [1, 16, 5])
    t2, l2 = from_csr(layout, indptr, indices, last, table_width=3)
    np.testing.assert_array_equal(l2, lengths)
    np.testing.assert_array_equal(t2, table)


@pytest.mark.parametrize("seed", range(5))
def test_round_trip_on_generated_metadata(seed):
    layout, table, lengths = make_metadata(7, 8, 2, 64, 700, 16, seed=seed)
    indptr, indices, last = paged_csr(layout, table, lengths)
    t2, l2 = from_csr(layout, indptr, indices, last, table_width=table.shape[1])
    np.testing.assert_array_equal(l2, lengths)
    live = (np.arange(table.shape[1])[None] * 16) < lengths[:, None]
    np.testing.assert_array_equal(np.where(live, t2, -1), np.where(live, table, -1))


def test_rejections():
    layout = Layout(2, 4, 2, 64, 16, 8)
    with pytest.raises(ValueError):
        paged_csr(layout, np.zeros((2, 2), np.int32), np.array([0, 3]))          # empty context
    with pytest.raises(ValueError):
        from_csr(layout, [0, 1, 3], [1, 2], [1, 1])                              # indptr end != nnz
    with pytest.raises(ValueError):
        from_csr(layout, [0, 1, 2], [1, 2], [0, 4])                              # last_page_len 0
    with pytest.raises(ValueError):
        from_csr(layout, [0, 1, 2], [1, 99], [1, 1])                             # page id out of range
    with pytest.raises(TypeError):
        from_csr(layout, [0.0, 1.0, 2.0], [1, 2], [1, 1])
    with pytest.raises(ValueError):
        from_csr(layout, [0, 2, 3], [1, 2, 3], [1, 1], table_width=1)           # width too small
    t, l = from_csr(layout, [0, 0, 1], [5], [1, 7])                               # empty first sequence
    np.testing.assert_array_equal(l, [0, 7])
    assert t.shape == (2, 1) and t[1, 0] == 5
