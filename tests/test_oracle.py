"""Pins the FP64 oracle (oracle/fp64.py) independently of its own formulas.

Mirrors reference tests/test_oracle.py:8-63 (split invariance, shared prefix
pages, the extreme-logit known-answer merge test) and adds checks that do not
reuse the oracle's expressions: a per-token brute force with math.exp/fsum,
closed forms (empty row, q = 0, one token), page relabelling and GQA == MHA.
"""
import math

import numpy as np
import pytest

from oracle import fp64
from paged_decode.layout import Layout
from paged_decode.workload import make_metadata


def brute_force(q, k, v, table, lengths):
    """Token-by-token softmax attention with Python floats (no NumPy reductions)."""
    batch, heads, dim = q.shape
    page_size, kv_heads = k.shape[1], k.shape[2]
    group = heads // kv_heads
    out = np.zeros((batch, heads, dim))
    for b in range(batch):
        for h in range(heads):
            scores, rows = [], []
            for t in range(int(lengths[b])):
                page = int(table[b][t // page_size])
                key = [float(x) for x in k[page, t % page_size, h // group]]
                rows.append([float(x) for x in v[page, t % page_size, h // group]])
                scores.append(math.fsum(float(a) * kk for a, kk in zip(q[b, h], key)) / math.sqrt(dim))
            if not scores:
                continue
            top = max(scores)
            weights = [math.exp(s - top) for s in scores]
            total = math.fsum(weights)
            for d in range(dim):
                out[b, h, d] = math.fsum(w * r[d] for w, r in zip(weights, rows)) / total
    return out


def small_problem(seed=4, dim=64, magnitude=1.0):
    layout, table, lengths = make_metadata(3, 4, 2, dim, 35, 16)
    lengths[:] = [0, 1, 35]
    table = np.random.default_rng(9).permutation(layout.physical_pages).reshape(3, -1)
    rng = np.random.default_rng(seed)
    q = rng.normal(size=(3, 4, dim)) * magnitude
    k = rng.normal(size=(layout.physical_pages, 16, 2, dim))
    v = rng.normal(size=k.shape)
    return q, k, v, table, lengths


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("split", [1, 17, 256])
@pytest.mark.parametrize("magnitude", [1.0, 100.0])
def test_partitioned_attention_matches_dense(dim, split, magnitude):
    q, k, v, table, lengths = small_problem(dim=dim, magnitude=magnitude)
    expected = fp64.dense_attention(q, k, v, table, lengths)
    actual = fp64.streaming_attention(q, k, v, table, lengths, split)
    np.testing.assert_allclose(actual, expected, rtol=1e-11, atol=1e-11)
    assert np.isfinite(actual).all()


@pytest.mark.parametrize("magnitude", [1.0, 30.0])
def test_dense_matches_token_loop_brute_force(magnitude):
    q, k, v, table, lengths = small_problem(seed=21, dim=64, magnitude=magnitude)
    np.testing.assert_allclose(fp64.dense_attention(q, k, v, table, lengths),
                               brute_force(q, k, v, table, lengths), rtol=1e-12, atol=1e-12)


def test_shared_prefix_pages():
    rng = np.random.default_rng(8)
    q = rng.normal(size=(2, 4, 64))
    k, v = rng.normal(size=(2, 3, 16, 2, 64))
    table = np.array([[2, 0], [2, 1]])
    lengths = np.array([17, 31])
    np.testing.assert_allclose(fp64.streaming_attention(q, k, v, table, lengths, 7),
                               fp64.dense_attention(q, k, v, table, lengths), atol=1e-12)
    np.testing.assert_allclose(fp64.dense_attention(q, k, v, table, lengths),
                               brute_force(q, k, v, table, lengths), atol=1e-12)


def test_softmax_merge_survives_extreme_logits_and_empty_partitions():
    # Known-answer vector of reference tests/test_oracle.py:55-63.
    scores = np.array([-10000., 10000., 9999.])
    values = np.arange(12, dtype=float).reshape(3, 4)
    parts = [fp64.partial_softmax(scores[:0], values[:0]),
             fp64.partial_softmax(scores[:1], values[:1]),
             fp64.partial_softmax(scores[1:], values[1:])]
    # Closed form: e^-20000 vanishes, so only the last two rows weigh in with
    # weights 1 : e^-1.
    w = math.exp(-1.0)
    expected = (values[1] + w * values[2]) / (1.0 + w)
    np.testing.assert_allclose(fp64.merge_partials(parts), expected, rtol=1e-15)
    np.testing.assert_array_equal(fp64.merge_partials(parts[:1]), np.zeros(4))


def test_partial_state_of_known_scores():
    m, l, n = fp64.partial_softmax([0.0, math.log(3.0)], [[1.0, 0.0], [0.0, 1.0]])
    assert m == pytest.approx(math.log(3.0))
    assert l == pytest.approx(1.0 + 1.0 / 3.0)
    np.testing.assert_allclose(n, [1.0 / 3.0, 1.0])


def test_empty_rows_are_zero_and_one_token_returns_its_value():
    q, k, v, table, lengths = small_problem(seed=5)
    out = fp64.dense_attention(q, k, v, table, lengths)
    np.testing.assert_array_equal(out[0], 0.0)           # length 0
    page = table[1][0]
    for h in range(4):                                   # length 1: exactly V of token 0
        np.testing.assert_allclose(out[1, h], v[page, 0, h // 2], rtol=1e-15)


def test_zero_query_gives_mean_of_values():
    q, k, v, table, lengths = small_problem(seed=6)
    q[:] = 0.0
    out = fp64.dense_attention(q, k, v, table, lengths)
    for h in range(4):
        live = np.stack([v[table[2][t // 16], t % 16, h // 2] for t in range(35)])
        np.testing.assert_allclose(out[2, h], live.mean(axis=0), rtol=1e-13, atol=1e-15)


def test_page_relabelling_is_invisible():
    q, k, v, table, lengths = small_problem(seed=7)
    perm = np.random.default_rng(1).permutation(k.shape[0])  # physical page p moves to perm[p]
    k2, v2 = np.empty_like(k), np.empty_like(v)
    k2[perm], v2[perm] = k, v
    table2 = perm[table]
    np.testing.assert_allclose(fp64.dense_attention(q, k2, v2, table2, lengths),
                               fp64.dense_attention(q, k, v, table, lengths), rtol=1e-14, atol=1e-15)


def test_gqa_equals_mha_over_repeated_kv_heads():
    q, k, v, table, lengths = small_problem(seed=8)
    k_mha, v_mha = np.repeat(k, 2, axis=2), np.repeat(v, 2, axis=2)
    np.testing.assert_allclose(fp64.dense_attention(q, k_mha, v_mha, table, lengths),
                               fp64.dense_attention(q, k, v, table, lengths), rtol=1e-14, atol=1e-15)


def test_gather_reads_pages_through_table():
    cache = np.arange(3 * 4 * 2 * 1, dtype=float).reshape(3, 4, 2, 1)  # value = ((p*4+t)*2+h)
    got = fp64.gather_tokens(cache, np.array([2, 0]), 6, kv_head=1)[:, 0]
    expected = [((2 * 4 + t) * 2 + 1) for t in range(4)] + [((0 * 4 + t) * 2 + 1) for t in range(2)]
    np.testing.assert_array_equal(got, expected)
    assert fp64.gather_tokens(cache, np.array([-1]), 0, 0).shape == (0, 1)


def test_padding_ids_past_live_prefix_are_never_read():
    q, k, v, table, lengths = small_problem(seed=9)
    padded = table.copy()
    padded[1, 1:] = -1          # length 1 uses one page
    np.testing.assert_allclose(fp64.dense_attention(q, k, v, padded, lengths),
                               fp64.dense_attention(q, k, v, table, lengths), rtol=0, atol=0)


def test_streaming_rejects_nonpositive_split():
    q, k, v, table, lengths = small_problem()
    with pytest.raises(ValueError):
        fp64.streaming_attention(q, k, v, table, lengths, 0)


def test_oracle_is_not_imported_by_the_product_package():
    import importlib
    import pathlib
    import sys

    root = pathlib.Path(importlib.import_module("paged_decode").__file__).parent
    for path in root.rglob("*.py"):
        text = path.read_text()
        assert "from oracle" not in text and "import oracle" not in text, path
    assert "oracle.fp64" in sys.modules  # only this test module imported it


def test_scatter_then_gather_round_trip():
    """Writing tokens and reading them back through the same table returns them."""
    rng = np.random.default_rng(21)
    pages, page_size, kv, dim = 12, 4, 2, 8
    cache = rng.standard_normal((pages, page_size, kv, dim))
    table = rng.permutation(pages).reshape(3, 4).astype(np.int32)
    new = rng.standard_normal((3, 5, kv, dim))
    positions = np.array([0, 3, 11], dtype=np.int32)
    out = fp64.scatter_tokens(cache, table, positions, new)
    for b in range(3):
        stop = min(positions[b] + 5, 16)
        got = np.stack([fp64.gather_tokens(out, table[b], stop, h)[positions[b]:] for h in range(kv)], axis=1)
        np.testing.assert_array_equal(got, new[b, :stop - positions[b]])
    written = {(int(table[b, p // page_size]), p % page_size)
               for b in range(3) for p in range(positions[b], min(positions[b] + 5, 16))}
    for page in range(pages):
        for slot in range(page_size):
            if (page, slot) not in written:
                np.testing.assert_array_equal(out[page, slot], cache[page, slot])


def test_scatter_skips_invalid_positions_and_pages():
    cache = np.zeros((4, 2, 1, 2))
    table = np.array([[0, -1], [9, 1]], dtype=np.int32)
    new = np.ones((2, 3, 1, 2))
    out = fp64.scatter_tokens(cache, table, np.array([-1, 1]), new)
    # seq 0: positions -1 (skip), 0 -> page 0 slot 0, 1 -> page 0 slot 1
    # seq 1: positions 1 (page 9, skip), 2 -> page 1 slot 0, 3 -> page 1 slot 1
    assert out[0].sum() == 4 and out[1].sum() == 4 and out[2:].sum() == 0


def test_append_advance_is_all_or_nothing():
    cache = np.zeros((4, 2, 1, 1))
    table = np.array([[0, 1], [2, -1]], dtype=np.int32)
    new = np.arange(1, 5, dtype=np.float64).reshape(2, 2, 1, 1)
    out, lengths = fp64.append_advance(cache, table, np.array([1, 1]), new)
    np.testing.assert_array_equal(lengths, [3, 1])          # seq 1 would need page -1
    assert out[0, 1, 0, 0] == 1 and out[1, 0, 0, 0] == 2 and out[2:].sum() == 0


def test_append_advance_stops_at_the_context_capacity():
    """A capacity below the table's refuses any append that would cross it,
    all or nothing, and leaves the cache untouched."""
    cache = np.zeros((4, 2, 1, 1))
    table = np.array([[0, 1], [2, 3]], dtype=np.int32)
    new = np.arange(1, 5, dtype=np.float64).reshape(2, 2, 1, 1)
    out, lengths = fp64.append_advance(cache, table, np.array([0, 1]), new, max_context=2)
    np.testing.assert_array_equal(lengths, [2, 1])          # seq 1 would reach position 2
    assert out[0, 0, 0, 0] == 1 and out[0, 1, 0, 0] == 2 and out[1:].sum() == 0
    same, lengths = fp64.append_advance(out, table, lengths, new, max_context=2)
    np.testing.assert_array_equal(lengths, [2, 1])
    np.testing.assert_array_equal(same, out)
    _, lengths = fp64.append_advance(cache, table, np.array([0, 1]), new, max_context=100)
    np.testing.assert_array_equal(lengths, [2, 3])          # above the table's 4: the table bounds it
