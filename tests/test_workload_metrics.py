"""Workload generators and timing summaries.

make_metadata is pinned by the lengths the reference's own benchmark reports
recorded for seed 123 (tests/golden/recorded_metadata.json). Metric cases
mirror reference tests/test_metrics.py:5-20.
"""
import json

import numpy as np
import pytest

from paged_decode.metrics import kv_bytes, percentile, summarize, unique_token_bytes
from paged_decode.workload import WORKLOAD_NAMES, make_metadata, make_workload


def test_make_metadata_reproduces_recorded_lengths(golden_dir):
    cases = json.loads((golden_dir / "recorded_metadata.json").read_text())
    assert len(cases) >= 9
    for case in cases:
        layout, table, lengths = make_metadata(case["batch"], case["heads"], case["kv_heads"], case["dim"],
                                               case["context"], case["page_size"], seed=case["seed"],
                                               ragged=not case["uniform"])
        assert lengths.tolist() == case["lengths"], case["source"]
        assert layout.physical_pages == case["physical_pages"], case["source"]
        live = (lengths + case["page_size"] - 1) // case["page_size"]
        for row, n in enumerate(live):
            assert np.all(table[row, :n] >= 0) and np.all(table[row, n:] == -1)
        assert np.unique(table[table >= 0]).size == (table >= 0).sum()  # one owner per page


def test_make_metadata_rejects_nonpositive():
    with pytest.raises(ValueError):
        make_metadata(0, 4, 2, 64, 16, 16)


@pytest.mark.parametrize("name", WORKLOAD_NAMES)
def test_named_workloads_are_valid(name):
    from paged_decode.layout import validate_metadata

    w = make_workload(name)
    validate_metadata(w.layout, w.table, w.lengths)
    assert w.table.dtype == np.int32 and w.lengths.dtype == np.int32


def test_named_workload_shapes():
    w = make_workload("llama3_8b_b4_l4096")
    assert (w.layout.batch, w.layout.query_heads, w.layout.kv_heads, w.layout.head_dim, w.layout.page_size) == \
        (4, 32, 8, 128, 16)
    assert kv_bytes(w.lengths, 8, 128, 2) == 67_108_864
    w = make_workload("ragged_shared_b16")
    assert (w.lengths == 0).any() and w.lengths.max() <= 8192 and w.split_tokens == 128
    shared = w.table[:, :64]
    live = shared >= 0
    assert np.all(shared[live] == np.broadcast_to(np.arange(64), shared.shape)[live])
    assert unique_token_bytes(w.table, w.lengths, 32, 8, 128, 2) < kv_bytes(w.lengths, 8, 128, 2)
    w = make_workload("mqa_b128_l1024")
    assert kv_bytes(w.lengths, 1, 64, 2) == 33_554_432
    q, k, v = w.host_tensors()
    assert 0.03 < (np.abs(k) > 6).mean() < 0.07   # ~5% of keys scaled x20
    w = make_workload("long_mha_b1_l32768")
    assert kv_bytes(w.lengths, 32, 128, 2) == 536_870_912 and w.split_sweep == (128, 256, 512, 1024)
    w = make_workload("fp32_b2_ragged")
    assert w.lengths.tolist() == [100, 256] and w.layout.physical_pages == 32


def test_reference_benchmark_workloads_use_the_recorded_lengths(golden_dir):
    """The reference's benchmark shape at B1/B4/B16 has the lengths its own reports recorded."""
    cases = json.loads((golden_dir / "recorded_metadata.json").read_text())
    recorded = {c["batch"]: c["lengths"] for c in cases
                if c["context"] == 4096 and not c["uniform"] and c["heads"] == 32 and c["page_size"] == 16}
    for batch in (1, 4, 16):
        w = make_workload(f"reference_b{batch}_l4096")
        assert w.lengths.tolist() == recorded[batch]
        assert (w.layout.query_heads, w.layout.kv_heads, w.layout.head_dim, w.split_tokens) == (32, 8, 128, 256)
    assert make_workload("reference_b4_l4096").lengths.tolist() == [4096, 2311, 2289, 2568]


def test_percentiles_are_interpolated():
    assert percentile([1, 2, 3, 4, 5], .95) == pytest.approx(4.8)
    assert percentile([5], .95) == 5
    assert percentile([3, 1, 2], 0.5) == 2


def test_percentiles_match_numpy_linear_method():
    rng = np.random.default_rng(7)
    for n in (1, 2, 3, 10, 31):
        sample = rng.standard_normal(n).tolist()
        for quantile in (0.0, 0.05, 0.5, 0.95, 1.0, 1 / 3):
            assert percentile(sample, quantile) == pytest.approx(np.percentile(sample, 100 * quantile), abs=1e-12)
    for bad in (-0.01, 1.01):
        with pytest.raises(ValueError):
            percentile([1.0], bad)
    with pytest.raises(ValueError):
        percentile([], 0.5)


def test_throughput_uses_sequences_per_decode_step():
    summary = summarize([1., 2., 3.], [2., 3., 4.], batch=8)
    assert summary["device_ms_p50"] == 2
    assert summary["sequence_tokens_per_second"] == 4000
    assert summary["wall_ms_p50"] == 3


@pytest.mark.parametrize("device,wall", [([], []), ([0.], [1.]), ([1.], [])])
def test_invalid_samples_are_rejected(device, wall):
    with pytest.raises(ValueError):
        summarize(device, wall, 1)


def test_unique_token_bytes_counts_shared_slots_once():
    table = np.array([[0, 1], [0, 2]])
    lengths = np.array([20, 17])
    # slots: seq0 page0 all 16 + page1 4; seq1 page0 16 (shared) + page2 1
    assert unique_token_bytes(table, lengths, 16, 1, 1, 1) == (16 + 4 + 1) * 2
    assert kv_bytes(lengths, 1, 1, 1) == 37 * 2
