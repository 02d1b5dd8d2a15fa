"""The C FP32 split-K restatement (oracle/cpu_decode.c) against the FP64 oracle.

It is the timed CPU baseline, so it must agree with the oracle to FP32
accumulation accuracy and share the GPU path's edge semantics.
"""
import numpy as np
import pytest

from oracle import cpu, fp64
from paged_decode.layout import Layout
from paged_decode.workload import host_tensors, make_workload


@pytest.mark.parametrize("dtype", [np.float32, np.float16])
@pytest.mark.parametrize("split", [1, 13, 64, 256])
def test_matches_fp64_oracle(dtype, split):
    layout = Layout(3, 8, 2, 64, 16, 24)
    table = np.random.default_rng(3).permutation(24).reshape(3, 8).astype(np.int32)
    lengths = np.array([0, 17, 127], dtype=np.int32)
    q, k, v = host_tensors(layout, dtype=dtype, seed=2)
    expected = fp64.dense_attention(q, k, v, table, lengths)
    actual = cpu.decode(q, k, v, table, lengths, split, threads=2)
    np.testing.assert_allclose(actual, expected, atol=2e-6, rtol=1e-5)
    np.testing.assert_array_equal(actual[0], 0.0)


@pytest.mark.parametrize("name", ["fp32_b2_ragged", "llama3_8b_b4_l4096", "mqa_b128_l1024"])
def test_named_workloads(name):
    w = make_workload(name)
    q, k, v = w.host_tensors()
    expected = fp64.dense_attention(q, k, v, w.table, w.lengths)
    actual = cpu.decode(q, k, v, w.table, w.lengths, w.split_tokens)
    np.testing.assert_allclose(actual, expected, atol=2e-5, rtol=1e-5)


def test_invalid_page_ids_are_skipped():
    layout = Layout(1, 2, 1, 64, 16, 2)
    q, k, v = host_tensors(layout, dtype=np.float32, seed=4)
    table = np.array([[0, 7]], dtype=np.int32)         # second live page is out of range
    lengths = np.array([20], dtype=np.int32)
    out = cpu.decode(q, k, v, table, lengths, 8, threads=1)
    expected = fp64.dense_attention(q, k, v, table[:, :1], np.array([16]))
    np.testing.assert_allclose(out, expected, atol=2e-6, rtol=1e-5)


def test_threads_do_not_change_results():
    w = make_workload("ragged_shared_b16")
    q, k, v = w.host_tensors()
    a = cpu.decode(q, k, v, w.table, w.lengths, w.split_tokens, threads=1)
    b = cpu.decode(q, k, v, w.table, w.lengths, w.split_tokens, threads=4)
    np.testing.assert_array_equal(a, b)


def test_rejects_mixed_dtypes():
    layout = Layout(1, 2, 1, 64, 16, 2)
    q, k, v = host_tensors(layout, dtype=np.float32)
    with pytest.raises(TypeError):
        cpu.decode(q.astype(np.float16), k, v, np.array([[0, 1]]), np.array([3]))
