"""CSR page-list metadata (engine format) <-> page table + lengths.

Engines such as FlashInfer describe a paged KV cache as three arrays:
``indptr [B+1]`` (page-list offsets), ``indices [nnz]`` (physical page ids in
logical order) and ``last_page_len [B]`` (tokens in each sequence's last page,
1..page_size). ``paged_csr`` produces them from a table and lengths with the
semantics of reference ``src/paged_decode/competitors.py:8-18``;
``from_csr`` is its inverse, so a caller holding CSR metadata can build a
``DecodePlan`` directly (``DecodePlan.from_csr``).
"""
import numpy as np

from .layout import Layout, validate_metadata


def paged_csr(layout: Layout, table, lengths):
    """``(indptr, indices, last_page_len)`` int32 arrays for nonempty sequences.

    Raises ``ValueError`` for an empty sequence (the format has no encoding for
    it) or when the page list would overflow int32, as the reference does.
    """
    table, lengths = validate_metadata(layout, table, lengths)
    if np.any(lengths == 0):
        raise ValueError("the CSR page-list format requires nonempty contexts")
    counts = (lengths.astype(np.int64) + layout.page_size - 1) // layout.page_size
    indptr = np.zeros(len(counts) + 1, dtype=np.int64)
    np.cumsum(counts, out=indptr[1:])
    if int(indptr[-1]) > np.iinfo(np.int32).max:
        raise ValueError("CSR page list exceeds int32 capacity")
    indices = np.concatenate([table[b, :int(c)] for b, c in enumerate(counts)]) if len(counts) else \
        np.zeros(0, dtype=np.int32)
    last = (lengths.astype(np.int64) - 1) % layout.page_size + 1
    return indptr.astype(np.int32), indices.astype(np.int32), last.astype(np.int32)


def from_csr(layout: Layout, indptr, indices, last_page_len, *, table_width=None):
    """``(table [B, W], lengths [B])`` int32 from CSR metadata.

    ``table_width`` defaults to the longest page list; rows are padded with
    ``-1``. A sequence with an empty page list gets length 0. The result is
    validated like any plan metadata (page ids in range, lengths within the
    table).
    """
    indptr = np.asarray(indptr)
    indices = np.asarray(indices)
    last = np.asarray(last_page_len)
    for name, arr in (("indptr", indptr), ("indices", indices), ("last_page_len", last)):
        if arr.dtype.kind not in "iu":
            raise TypeError(f"{name} must be an integer array")
    if indptr.shape != (layout.batch + 1,) or last.shape != (layout.batch,) or indices.ndim != 1:
        raise ValueError("expected indptr [B+1], indices [nnz], last_page_len [B]")
    counts = np.diff(indptr.astype(np.int64))
    if indptr[0] != 0 or np.any(counts < 0) or int(indptr[-1]) != indices.shape[0]:
        raise ValueError("indptr must start at 0, be non-decreasing and end at len(indices)")
    if np.any((counts > 0) & ((last < 1) | (last > layout.page_size))):
        raise ValueError("last_page_len must be in [1, page_size] for nonempty page lists")
    width = int(counts.max(initial=0)) if table_width is None else int(table_width)
    if width < max(1, int(counts.max(initial=0))):
        raise ValueError("table_width is smaller than the longest page list")
    table = np.full((layout.batch, width), -1, dtype=np.int64)
    for b in range(layout.batch):
        table[b, :counts[b]] = indices[indptr[b]:indptr[b + 1]]
    lengths = np.where(counts > 0, (counts - 1) * layout.page_size + last.astype(np.int64), 0)
    return validate_metadata(layout, table, lengths)
