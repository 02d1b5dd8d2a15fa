"""Layout and metadata validation (product host logic).

Mirrors the validation cases of reference tests/test_oracle.py:26-42 and
:66-90 against paged_decode.layout, plus the drop-in import path.
"""
import numpy as np
import pytest

from paged_decode.layout import Layout, validate_metadata


def test_drop_in_import_path():
    from paged_decode.oracle import Layout as L2, validate_metadata as v2

    assert L2 is Layout and v2 is validate_metadata


@pytest.mark.parametrize("bad_lengths", [[-1, 1], [33, 1]])
def test_invalid_lengths_rejected(bad_lengths):
    layout = Layout(2, 4, 2, 64, 16, 4)
    with pytest.raises(ValueError):
        validate_metadata(layout, np.array([[0, 1], [2, 3]]), np.array(bad_lengths))


def test_padding_is_not_a_live_page():
    layout = Layout(1, 4, 2, 64, 16, 2)
    table, lengths = validate_metadata(layout, np.array([[0, -1]]), np.array([1]))
    assert table.dtype == lengths.dtype == np.int32
    with pytest.raises(ValueError):
        validate_metadata(layout, np.array([[0, -1]]), np.array([17]))
    with pytest.raises(ValueError):
        validate_metadata(layout, np.array([[2, 0]]), np.array([1]))
    with pytest.raises(TypeError):
        validate_metadata(layout, np.array([[0., 1.]]), np.array([1]))


def test_shape_checks():
    layout = Layout(2, 4, 2, 64, 16, 4)
    with pytest.raises(ValueError):
        validate_metadata(layout, np.array([0, 1]), np.array([1, 1]))          # 1-D table
    with pytest.raises(ValueError):
        validate_metadata(layout, np.array([[0, 1]]), np.array([1, 1]))        # wrong batch
    with pytest.raises(ValueError):
        validate_metadata(layout, np.array([[0], [1]]), np.array([1]))         # lengths shape
    with pytest.raises(TypeError):
        validate_metadata(layout, np.array([[0], [1]]), np.array([True, False]))


def test_unsigned_and_wide_integer_metadata_accepted():
    layout = Layout(1, 4, 2, 64, 16, 2)
    table, lengths = validate_metadata(layout, np.array([[1, 0]], dtype=np.uint64), np.array([20], dtype=np.int64))
    np.testing.assert_array_equal(table, [[1, 0]])
    assert lengths[0] == 20 and lengths.dtype == np.int32


def test_metadata_validation_copies_caller_arrays():
    layout = Layout(1, 4, 2, 64, 16, 2)
    table, lengths = np.array([[0, 1]]), np.array([17])
    copied_table, copied_lengths = validate_metadata(layout, table, lengths)
    table[:] = -1
    lengths[:] = 0
    np.testing.assert_array_equal(copied_table, [[0, 1]])
    np.testing.assert_array_equal(copied_lengths, [17])


@pytest.mark.parametrize("value", [True, False, 1.5, "4", np.float64(4)])
def test_layout_requires_integer_dimensions(value):
    with pytest.raises(TypeError):
        Layout(value, 4, 2, 64, 16, 2)


@pytest.mark.parametrize("value", [0, -1])
def test_layout_requires_positive_dimensions(value):
    with pytest.raises(ValueError):
        Layout(value, 4, 2, 64, 16, 2)


def test_invalid_head_ratio_is_rejected():
    with pytest.raises(ValueError):
        Layout(1, 3, 2, 64, 16, 2)


def test_numpy_integers_and_group():
    layout = Layout(np.int64(2), 32, np.int32(8), 128, 16, 4)
    assert layout.group == 4
