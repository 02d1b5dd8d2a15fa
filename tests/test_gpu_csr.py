"""Device-side CSR page lists -> page table and lengths (pd_table_from_csr).

Parity is by round trip: ``paged_csr`` (reference competitors.py:8-18
semantics, pinned in tests/test_csr.py) turns a table and lengths into CSR,
and the device conversion must give back exactly that table (with -1 padding)
and those lengths. Overflowing rows are checked against the documented rule,
and a captured refresh + decode graph against the FP64 oracle.
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode.csr import paged_csr  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import make_metadata, make_tensors  # noqa: E402

pytestmark = pytest.mark.gpu


def device(*arrays):
    return tuple(torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda() for a in arrays)


def csr_with_empty_rows(layout, table, lengths):
    """CSR of (table, lengths) where some lengths are 0 (paged_csr rejects those)."""
    counts = (lengths + layout.page_size - 1) // layout.page_size
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    indices = np.concatenate([table[b, :c] for b, c in enumerate(counts)]).astype(np.int32)
    last = np.where(lengths > 0, (lengths - 1) % layout.page_size + 1, 0).astype(np.int32)
    return indptr, indices, last


@pytest.mark.parametrize("batch,context,page_size,seed", [(4, 4096, 16, 123), (16, 4096, 32, 7), (3, 1000, 16, 1)])
def test_device_csr_round_trip(batch, context, page_size, seed):
    announce(f"device csr round trip B{batch} L{context} T{page_size}")
    layout, table, lengths = make_metadata(batch, 8, 2, 64, context, page_size, seed=seed)
    indptr, indices, last = paged_csr(layout, table, lengths)
    plan = DecodePlan(layout, table, np.zeros_like(lengths), max_context=context)
    plan._table.fill_(12345)
    overflow = torch.zeros(1, dtype=torch.int32, device="cuda")
    plan.refresh_csr(*device(indptr, indices, last), overflow=overflow)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(plan._table.cpu().numpy(), table)
    np.testing.assert_array_equal(plan._lengths.cpu().numpy(), lengths)
    assert int(overflow.item()) == 0


def test_device_csr_empty_rows_and_overflow():
    announce("device csr empty rows and overflow")
    layout = Layout(6, 8, 2, 64, 16, 6 * 8)
    table = np.arange(6 * 8, dtype=np.int32).reshape(6, 8)
    lengths = np.array([0, 128, 17, 1, 0, 100], dtype=np.int32)
    for b, n in enumerate(lengths):
        table[b, (n + 15) // 16:] = -1
    indptr, indices, last = csr_with_empty_rows(layout, table, lengths)
    plan = DecodePlan(layout, table, lengths, max_context=128)
    overflow = torch.zeros(1, dtype=torch.int32, device="cuda")
    plan.refresh_csr(*device(indptr, indices, last), overflow=overflow)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(plan._table.cpu().numpy(), table)
    np.testing.assert_array_equal(plan._lengths.cpu().numpy(), lengths)
    assert int(overflow.item()) == 0

    # On a plan reserving 64 tokens: row 1 gets a last-page length outside
    # [1, page_size], row 2 a length above the reserved context; the other
    # rows convert normally.
    small = DecodePlan(layout, table, np.minimum(lengths, 64), max_context=64)
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    indptr2, indices2, last2 = csr_with_empty_rows(layout, table, np.array([0, 20, 100, 1, 0, 50], np.int32))
    last2[1] = 17
    small.refresh_csr(*device(indptr2, indices2, last2), overflow=flag)
    torch.cuda.synchronize()
    got_t, got_l = small._table.cpu().numpy(), small._lengths.cpu().numpy()
    assert int(flag.item()) == 1
    assert got_l.tolist() == [0, 0, 0, 1, 0, 50]               # rows 1 (bad last) and 2 (100 > 64) empty
    assert np.all(got_t[1] == -1) and np.all(got_t[2] == -1)
    np.testing.assert_array_equal(got_t[3, :1], table[3, :1])
    np.testing.assert_array_equal(got_t[5, :4], table[5, :4])
    assert np.all(got_t[5, 4:] == -1)

    # More pages than the table holds.
    wide = np.arange(20, dtype=np.int32)
    indptr3 = np.array([0, 0, 20, 20, 20, 20, 20], dtype=np.int32)   # row 1 has 20 pages > width 8
    flag.zero_()
    small.refresh_csr(*device(indptr3, wide, np.full(6, 16, np.int32)), overflow=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1 and small._lengths.cpu().numpy().tolist() == [0] * 6


def test_device_csr_page_lists_reaching_past_indices_are_not_read():
    """A malformed indptr whose page list reaches past the indices tensor (or
    starts before it) gives an empty row and raises the overflow flag instead
    of reading outside indices; well-formed rows convert normally."""
    announce("device csr: page lists outside the indices tensor")
    layout = Layout(4, 8, 2, 64, 16, 4 * 8)
    table = np.arange(4 * 8, dtype=np.int32).reshape(4, 8)
    lengths = np.array([128, 64, 16, 128], dtype=np.int32)
    for b, n in enumerate(lengths):
        table[b, (n + 15) // 16:] = -1
    indptr, indices, last = csr_with_empty_rows(layout, table, lengths)
    plan = DecodePlan(layout, table, lengths, max_context=128)
    bad = indptr.copy()
    bad[3] = -5                     # row 2: a negative page count; row 3: starts before indices ...
    bad[4] = indices.size + 5       # ... and ends past its last entry. Both rows are rejected.
    flag = torch.zeros(1, dtype=torch.int32, device="cuda")
    plan.refresh_csr(*device(bad, indices, last), overflow=flag)
    torch.cuda.synchronize()
    got_t, got_l = plan._table.cpu().numpy(), plan._lengths.cpu().numpy()
    assert int(flag.item()) == 1
    assert got_l.tolist() == [128, 64, 0, 0]
    np.testing.assert_array_equal(got_t[:2], table[:2])
    assert np.all(got_t[2:] == -1)


@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_captured_csr_refresh_then_decode(merge):
    """One graph = load this step's CSR page lists, then decode; replayed after the lists change."""
    announce(f"captured csr refresh + decode merge={merge}")
    layout = Layout(3, 8, 2, 128, 16, 3 * 16)
    q, k, v = make_tensors(layout, seed=19)
    rng = np.random.default_rng(2)
    table0 = rng.permutation(48).reshape(3, 16).astype(np.int32)
    plan = DecodePlan(layout, table0, np.array([256, 256, 256], np.int32), split_tokens=64, merge=merge)
    nnz = 3 * 16
    d_indptr = torch.zeros(4, dtype=torch.int32, device="cuda")
    d_indices = torch.zeros(nnz, dtype=torch.int32, device="cuda")
    d_last = torch.zeros(3, dtype=torch.int32, device="cuda")
    plan.run(q, k, v)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            plan.refresh_csr(d_indptr, d_indices, d_last)
            out = plan.run(q, k, v)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    qh, kh, vh = (t.cpu().numpy() for t in (q, k, v))
    for step in range(4):
        lengths = rng.integers(1, 257, size=3).astype(np.int32)
        table = rng.permutation(48).reshape(3, 16).astype(np.int32)
        indptr, indices, last = paged_csr(layout, table, lengths)
        padded = np.zeros(nnz, np.int32)
        padded[:indices.size] = indices
        d_indptr.copy_(torch.from_numpy(indptr))
        d_indices.copy_(torch.from_numpy(padded))
        d_last.copy_(torch.from_numpy(last))
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(out.cpu().numpy(), dense_attention(qh, kh, vh, table, lengths), torch.float16)
