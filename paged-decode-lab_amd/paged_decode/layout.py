"""Cache layout record and host-side metadata validation.

Restates the contract of reference ``src/paged_decode/oracle.py:11-47``
(``Layout`` and ``validate_metadata``): the same checks, in the same order,
raising the same exception types. These run on the CPU once, when a plan is
built, so the device kernels never see unvalidated page ids from the public API.
"""
from dataclasses import dataclass
from numbers import Integral

import numpy as np

_INT32_MAX = int(np.iinfo(np.int32).max)


@dataclass(frozen=True)
class Layout:
    """Shapes of one paged decode problem.

    ``k``/``v`` are ``[physical_pages, page_size, kv_heads, head_dim]``, ``q`` is
    ``[batch, query_heads, head_dim]``. Query head ``h`` reads KV head
    ``h // (query_heads // kv_heads)``. Follows reference ``oracle.py:11-27``.
    """

    batch: int
    query_heads: int
    kv_heads: int
    head_dim: int
    page_size: int
    physical_pages: int

    def __post_init__(self):
        values = tuple(vars(self).values())
        for value in values:
            # bool is an Integral subclass; the reference rejects it explicitly.
            if isinstance(value, (bool, np.bool_)) or not isinstance(value, Integral):
                raise TypeError("layout dimensions must be integers, not booleans")
        if min(int(value) for value in values) <= 0:
            raise ValueError("layout dimensions must be positive")
        if self.query_heads % self.kv_heads != 0:
            raise ValueError("query_heads must be divisible by kv_heads")

    @property
    def group(self) -> int:
        """Query heads per KV head (1 = MHA, query_heads = MQA)."""
        return self.query_heads // self.kv_heads


def validate_metadata(layout, table, lengths):
    """Check a page table and sequence lengths; return int32 copies.

    ``table`` is ``[batch, logical_pages]``; entries past a sequence's live
    prefix may be any value (``-1`` by convention). ``lengths`` is ``[batch]``
    with ``0 <= length <= logical_pages * page_size``. Every live logical page
    must map into ``[0, physical_pages)``. Follows reference ``oracle.py:30-47``.
    """
    table = np.asarray(table)
    lengths = np.asarray(lengths)
    if table.ndim != 2 or table.shape[0] != layout.batch:
        raise ValueError("page table must have shape [batch, logical_pages]")
    if lengths.shape != (layout.batch,):
        raise ValueError("lengths must have shape [batch]")
    if table.dtype.kind not in "iu" or lengths.dtype.kind not in "iu":
        raise TypeError("metadata must contain integers")
    width = table.shape[1]
    wide_lengths = lengths.astype(np.int64)
    if np.any(wide_lengths < 0) or np.any(wide_lengths > width * layout.page_size):
        raise ValueError("sequence length exceeds page table capacity")
    if max(width, layout.physical_pages) > _INT32_MAX:
        raise ValueError("metadata exceeds int32 addressing limits")
    live_pages = (wide_lengths + layout.page_size - 1) // layout.page_size
    live = np.arange(width, dtype=np.int64)[None, :] < live_pages[:, None]
    ids = table.astype(np.int64) if table.dtype.kind == "i" else table.astype(np.uint64)
    outside = (ids < 0) | (ids >= layout.physical_pages)
    if np.any(live & outside):
        raise ValueError("live logical page maps outside physical cache")
    return table.astype(np.int32, copy=True), lengths.astype(np.int32, copy=True)
