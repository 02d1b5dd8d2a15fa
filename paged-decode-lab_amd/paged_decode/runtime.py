"""Validated, allocation-free replay API over the gfx950 decode kernels.

``DecodePlan`` keeps the constructor, attributes, validation order, exception
types and borrowed-output contract of reference
``src/paged_decode/runtime.py:23-90``. Underneath, ``run`` makes one call into
the ``_C`` PyTorch extension, which launches the HIP kernels of
``libpaged_decode_hip.so`` on the current stream. There is no CPU or eager
fallback: if the native libraries cannot be loaded, plan construction fails.
"""
from functools import lru_cache
import importlib
import math

import numpy as np
import torch

from .layout import Layout, validate_metadata

# Four (m, l, n[D]) states per partition (one per quarter) and query head, as
# in the reference's workspace (runtime.py:64-68). The LDS-bounded merge holds
# one float per state, so "shared" becomes "serial_fallback" above 4096 states
# (runtime.py:54).
_STATES_PER_SPLIT = 4
_SHARED_MERGE_MAX_PARTS = 4096


@lru_cache(maxsize=1)
def load_extension():
    """Load the prebuilt extension; build it in-tree first if it is missing.

    Never called on import: plan construction is where native code is first
    touched (reference ``runtime.py:9-20``), so compilation and loading stay
    out of timed regions and graph capture. A process that has already
    initialised the GPU gets a RuntimeError instead of a build: compilers
    are child processes, which such a process must not start.
    """
    from . import _build

    if not _build.built():
        _build.refuse_after_gpu_init("building the missing paged_decode native libraries")
        _build.build()
    try:
        extension = importlib.import_module(f"{__package__}._C")
    except ImportError as exc:  # pragma: no cover - exercised only on broken installs
        raise RuntimeError(f"paged_decode native extension failed to load: {exc}") from exc
    _build.check_loaded(extension)
    return extension


class DecodePlan:
    """A decode problem prepared once and replayed many times.

    Construction validates the host page table and lengths, copies them to the
    device, and allocates the partition-state workspace and the output: ``run``
    then only launches kernels (no allocation, copy or synchronisation), so it
    can be timed or captured in a graph. q and the K/V cache are passed to
    every ``run`` and may hold new values each time; the metadata may change
    in place within the plan's shape and reserved context (``max_context``,
    default: the longest initial sequence) through ``refresh`` (host arrays),
    ``refresh_csr`` (CSR page lists on the device) or ``append`` (new tokens,
    lengths advanced on the device). Any other change needs a new plan.

    ``run`` returns the plan's own output tensor; the next ``run`` overwrites
    it, so copy it to keep it. The workspace and device metadata belong to the
    plan: callers must not modify them, and one plan serves one stream at a
    time (concurrent streams need separate plans).
    """

    def __init__(self, layout: Layout, table, lengths, *, device="cuda", split_tokens=256, merge="serial",
                 max_context=None):
        if merge not in ("serial", "shared"):
            raise ValueError("merge must be 'serial' or 'shared'")
        if layout.head_dim not in (64, 128):
            raise ValueError("head_dim must be 64 or 128")
        if layout.page_size not in (16, 32):
            raise ValueError("page_size must be 16 or 32")
        if layout.batch > 65535 or layout.query_heads > 65535:
            raise ValueError("batch/head count exceeds grid limits")
        if isinstance(split_tokens, bool) or not isinstance(split_tokens, int) or not 1 <= split_tokens <= 1048576:
            raise ValueError("split_tokens must be an integer in [1,1048576]")
        table, lengths = validate_metadata(layout, table, lengths)
        if table.shape[1] > 65536:
            raise ValueError("page table width must not exceed 65536")
        self.max_context = int(lengths.max(initial=0))
        if max_context is None:
            capacity = self.max_context
        else:
            if isinstance(max_context, bool) or not isinstance(max_context, int):
                raise ValueError("max_context must be an integer")
            if not self.max_context <= max_context <= table.shape[1] * layout.page_size:
                raise ValueError("max_context must cover the current lengths and fit the page table")
            capacity = max_context
        if capacity > 1048576:
            raise ValueError("this implementation supports at most 1M context tokens")
        self.context_capacity = capacity
        self.splits = max(1, math.ceil(capacity / split_tokens))
        if self.splits > 65535:
            raise ValueError("too many context splits")
        self.layout, self.split_tokens = layout, split_tokens
        self.merge = merge
        if merge == "shared":
            fits = self.splits * _STATES_PER_SPLIT <= _SHARED_MERGE_MAX_PARTS
            self.merge_implementation = "shared" if fits else "serial_fallback"
        else:
            self.merge_implementation = "serial"
        self._merge_mode = int(self.merge_implementation == "shared")
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("DecodePlan requires a GPU (torch 'cuda') device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        self._table_cpu, self._lengths_cpu = table, lengths
        self._unshared_pages = unshared_pages(table, layout.page_size, capacity)
        self._ragged_lengths = ragged_lengths(lengths)
        self._table = torch.tensor(table, device=self.device)
        self._lengths = torch.tensor(lengths, device=self.device)
        # Host-side upper bounds on the device lengths: the library launches
        # only the partitions they reach (ragged-batch compaction), plus a few
        # workgroups for lengths that grew further on the device.
        self._bounds = torch.from_numpy(lengths.astype(np.int32, copy=True))
        self._bounds_known = True
        shape = (layout.batch, layout.query_heads, self.splits * _STATES_PER_SPLIT)
        self._numerator = torch.empty((*shape, layout.head_dim), device=self.device, dtype=torch.float32)
        self._stats = torch.empty((*shape, 2), device=self.device, dtype=torch.float32)
        self._out = torch.empty((layout.batch, layout.query_heads, layout.head_dim),
                                dtype=torch.float32, device=self.device)
        self._stage_views = {}
        self._staged_split = (self.splits, split_tokens)
        self._extension = load_extension()
        self._prefix_runs = self._shared_prefixes(table)

    @classmethod
    def from_csr(cls, layout: Layout, indptr, indices, last_page_len, **kwargs):
        """Plan from CSR page-list metadata (``indptr``, ``indices``, ``last_page_len``).

        Same keyword arguments as the constructor; the table width is the
        longest page list unless ``table_width`` is given.
        """
        from .csr import from_csr

        table, lengths = from_csr(layout, indptr, indices, last_page_len, table_width=kwargs.pop("table_width", None))
        return cls(layout, table, lengths, **kwargs)

    def refresh(self, table, lengths):
        """Replace the page table and lengths in place, without reallocating.

        The new metadata is validated like the constructor's, must keep the
        table's shape, and its longest sequence must fit the plan's reserved
        context (``max_context`` at construction, else the first lengths).
        Partitions, workspace and device pointers are unchanged, so graphs
        captured from ``run`` stay valid and see the new metadata. The copy is
        ordered on the current stream: call it on the stream the plan runs on,
        outside graph capture.
        """
        table, lengths = validate_metadata(self.layout, table, lengths)
        if tuple(table.shape) != tuple(self._table.shape):
            raise ValueError("refresh must keep the page table shape")
        longest = int(lengths.max(initial=0))
        if longest > self.context_capacity:
            raise ValueError("lengths exceed the plan's reserved context; build a plan with a larger max_context")
        self._table.copy_(torch.from_numpy(table))
        self._lengths.copy_(torch.from_numpy(lengths))
        self._bounds.copy_(torch.from_numpy(lengths))
        self._bounds_known = True
        self._table_cpu, self._lengths_cpu = table, lengths
        self._unshared_pages = unshared_pages(table, self.layout.page_size, self.context_capacity)
        self._ragged_lengths = ragged_lengths(lengths)
        self._prefix_runs = self._shared_prefixes(table)
        self.max_context = longest

    def refresh_csr(self, indptr, indices, last_page_len, overflow=None):
        """Load CSR page-list metadata that lives on the device, without a host round trip.

        ``indptr [B+1]``, ``indices [nnz]`` and ``last_page_len [B]`` are
        contiguous int32 tensors on the plan device (the form
        ``paged_decode.csr.paged_csr`` produces). They are converted on the
        current stream into the plan's page table and lengths, so the call can
        be captured in a graph together with ``run``. A sequence whose page
        list is longer than the table or whose length exceeds the reserved
        context is loaded as empty and sets ``overflow[0]`` to 1 when an int32
        ``overflow`` tensor is given (it is never cleared; zero it first).
        Page ids are not validated here; the kernel skips ids outside the
        cache. ``max_context`` keeps the value of the last host-side metadata.
        The plan no longer knows whether pages are shared between sequences
        or how ragged the lengths are, so later runs keep K/V cacheable and
        the default workgroups (see ``unshared_pages``, ``ragged_lengths``).
        """
        for t in (indptr, indices, last_page_len):
            if t.device != self.device or t.dtype != torch.int32 or not t.is_contiguous():
                raise TypeError("CSR metadata must be contiguous int32 tensors on the plan device")
        if tuple(indptr.shape) != (self.layout.batch + 1,) or tuple(last_page_len.shape) != (self.layout.batch,) \
                or indices.dim() != 1:
            raise ValueError("expected indptr [B+1], indices [nnz], last_page_len [B]")
        if overflow is not None and (overflow.device != self.device or overflow.dtype != torch.int32):
            raise TypeError("overflow must be an int32 tensor on the plan device")
        self._extension.table_from_csr(indptr, indices, last_page_len, self._table, self._lengths, overflow,
                                       self.layout.page_size, self.context_capacity)
        self._unshared_pages = False
        self._ragged_lengths = False
        self._bounds_known = False
        self._prefix_runs = None

    def append(self, k_cache, v_cache, k_new, v_new):
        """Append new tokens at the plan's current lengths and advance them on the device.

        ``k_new``/``v_new`` are ``[B, Hkv, D]`` (one token per sequence) or
        ``[B, tokens, Hkv, D]``; the cache tensors are those later passed to
        ``run``. A sequence is written only if all of its new positions fall on
        valid pages of the plan's table below ``context_capacity`` (the
        reserved ``max_context``, which the plan's partitions cover);
        otherwise it and its length are unchanged, so a plan built without
        ``max_context`` above its longest sequence never grows that sequence. No host synchronisation: an append and
        a ``run`` can be captured together in one graph. ``max_context`` keeps
        the value of the last host-side metadata (construction or ``refresh``).
        """
        layout = self.layout
        expected_k = (layout.physical_pages, layout.page_size, layout.kv_heads, layout.head_dim)
        k_new, v_new = _token_batch(k_new, v_new, layout)
        _check_cache(k_cache, v_cache, k_new, v_new, expected_k, self.device)
        if k_new.shape[1] > self.context_capacity:
            raise ValueError("more new tokens than the plan's reserved context")
        self._extension.append_kv(k_new, v_new, self._table, self._lengths, k_cache, v_cache, True,
                                  self.context_capacity)
        if self._bounds_known:
            self._bounds.add_(k_new.shape[1]).clamp_(max=self.context_capacity)

    @property
    def workspace_bytes(self):
        """Bytes of the partition-state workspace (numerator + stats)."""
        return sum(t.numel() * t.element_size() for t in (self._numerator, self._stats))

    def _check(self, q, k, v, k_scale, v_scale):
        layout = self.layout
        expected_q = (layout.batch, layout.query_heads, layout.head_dim)
        expected_k = (layout.physical_pages, layout.page_size, layout.kv_heads, layout.head_dim)
        if tuple(q.shape) != expected_q or tuple(k.shape) != expected_k or tuple(v.shape) != expected_k:
            raise ValueError("input shape does not match plan")
        _check_formats(q.dtype, k.dtype, v.dtype)
        for scale in (k_scale, v_scale):
            if isinstance(scale, bool) or not isinstance(scale, (int, float)) or not 0 < scale < math.inf:
                raise ValueError("k_scale and v_scale must be finite and positive")
        for tensor in (q, k, v):
            if tensor.device != self.device or not tensor.is_contiguous():
                raise ValueError("inputs must be contiguous on the plan device")
            if tensor.requires_grad:
                raise ValueError("inference only: detach tensors requiring gradients")

    def run(self, q, k, v, *, k_scale=1.0, v_scale=1.0):
        """Decode one token per sequence; returns the borrowed FP32 [B, Hq, D] output.

        q, k, v share float16, bfloat16 or float32; k and v may instead be
        float8_e4m3fn or float8_e5m2 with a float16/bfloat16 q. The attention
        runs over ``k_scale * k`` and ``v_scale * v`` (per-tensor scales of a
        quantized cache; 1.0 for the reference's unscaled inputs).
        """
        self._check(q, k, v, k_scale, v_scale)
        self._extension.decode(q, k, v, self._table, self._lengths, self._numerator, self._stats,
                               self._out, self.split_tokens, self._merge_mode, float(k_scale), float(v_scale),
                               self._unshared_pages, self._ragged_lengths, self._length_bounds(), self._prefix_runs)
        return self._out

    def launches(self, q_dtype, kv_dtype=None):
        """Kernel launches ``run`` makes for q (and K/V) of these dtypes: 1 when the
        rows are small enough for one whole-row launch that writes the output
        (the workspace is then left unwritten), else 2 (partition, merge)."""
        layout = self.layout
        return self._extension.launch_count(q_dtype, q_dtype if kv_dtype is None else kv_dtype, layout.batch,
                                            layout.query_heads, layout.kv_heads, layout.head_dim, layout.page_size,
                                            self._table.shape[1], layout.physical_pages, self.splits,
                                            self.split_tokens, self._unshared_pages, self._ragged_lengths)

    def kernel_split(self, q_dtype, kv_dtype=None):
        """``(partitions, tokens per partition)`` per row that ``run``'s launches use
        for q (and K/V) of these dtypes at the current host length bounds: the
        plan's ``(splits, split_tokens)``, or on grids with many waves per CU a
        coarser split (a power of two times ``split_tokens``, with fewer
        partitions, so the workspace holds their states). With shared-prefix
        runs the split can be half the one the same call takes without them,
        so it comes from the launch plan."""
        layout = self.layout
        if self._prefix_runs is not None:
            return tuple(self.launch_plan(q_dtype, kv_dtype)["kernel_split"])
        return self._extension.kernel_split(q_dtype, q_dtype if kv_dtype is None else kv_dtype, layout.batch,
                                            layout.query_heads, layout.kv_heads, layout.head_dim, layout.page_size,
                                            self._table.shape[1], layout.physical_pages, self.splits,
                                            self.split_tokens, self._length_bounds())

    def launch_plan(self, q_dtype, kv_dtype=None, compute_units=0):
        """The launches ``run`` makes for q (and K/V) of these dtypes at the current
        host length bounds and hints: a dict with the launch count, the kernel
        split, the partition grid and workgroup shape, the grid kind, XCD
        grouping, quarter combine, streaming loads and the merge kernel
        variant (``pd_decode_launch_plan``). ``compute_units`` <= 0 means the
        current device's."""
        layout = self.layout
        return self._extension.launch_plan(q_dtype, q_dtype if kv_dtype is None else kv_dtype, layout.batch,
                                           layout.query_heads, layout.kv_heads, layout.head_dim, layout.page_size,
                                           self._table.shape[1], layout.physical_pages, self.splits,
                                           self.split_tokens, self._merge_mode, self._unshared_pages,
                                           self._ragged_lengths, self._length_bounds(), compute_units,
                                           self._prefix_runs)

    def _stage_workspace(self, splits):
        """Numerator and stats views for ``splits`` partitions per row: the leading
        part of the workspace buffers, as the full call uses them."""
        views = self._stage_views.get(splits)
        if views is None:
            layout = self.layout
            shape = (layout.batch, layout.query_heads, splits * _STATES_PER_SPLIT)
            states = math.prod(shape)
            views = (self._numerator.view(-1)[:states * layout.head_dim].view(*shape, layout.head_dim),
                     self._stats.view(-1)[:states * 2].view(*shape, 2))
            self._stage_views[splits] = views
        return views

    def run_partial(self, q, k, v, *, k_scale=1.0, v_scale=1.0):
        """Partition stage only (fills the workspace with the states; never a
        whole-row launch), over the partitions ``run``'s launches use
        (``kernel_split``); for stage timing."""
        self._check(q, k, v, k_scale, v_scale)
        splits, split_tokens = self.kernel_split(q.dtype, k.dtype)
        numerator, stats = self._stage_workspace(splits)
        self._extension.partial(q, k, v, self._table, self._lengths, numerator, stats, split_tokens,
                                float(k_scale), float(v_scale), self._unshared_pages, self._ragged_lengths,
                                self._length_bounds(), self._prefix_runs)
        self._staged_split = (splits, split_tokens)

    def _length_bounds(self):
        """Host upper bounds on the device lengths, or None after a device-side CSR refresh."""
        return self._bounds if self._bounds_known else None

    def _shared_prefixes(self, table):
        """Shared-prefix runs of the host table (``pd_prefix_runs``), or None when
        no page is mapped twice. With them, a work-list launch scores each
        partition inside several sequences' common prefix once for up to 16 / GT
        of them (one read of its K and V). The kernel checks the pages itself,
        so runs that no longer describe the device table (a graph captured
        before ``refresh``) cost time, never correctness."""
        if self._unshared_pages:
            return None
        return self._extension.prefix_runs(torch.from_numpy(np.ascontiguousarray(table, dtype=np.int32)))

    def run_merge(self):
        """Merge stage only, from the states the last ``run_partial`` left in the
        workspace (over its partitions); returns the borrowed output."""
        layout = self.layout
        splits, split_tokens = self._staged_split
        numerator, stats = self._stage_workspace(splits)
        self._extension.merge(numerator, stats, self._out, self._lengths, layout.page_size, self._table.shape[1],
                              split_tokens, self._merge_mode)
        return self._out


def unshared_pages(table, page_size, capacity):
    """True when no physical page is mapped twice among the table entries that
    can hold live tokens: columns up to ``ceil(capacity / page_size)`` of every
    row (appends can extend a sequence that far), negative padding excluded.

    The plan passes this as the library's page-sharing hint: with no page read
    twice, the partition kernel may stream K/V past the caches; with shared
    (prefix) pages it keeps them cacheable. Results are the same either way.
    """
    columns = min(table.shape[1], -(-int(capacity) // page_size))
    ids = np.asarray(table)[:, :columns].ravel()
    ids = ids[ids >= 0]
    return bool(np.unique(ids).size == ids.size)


def ragged_lengths(lengths):
    """True when the batch's live tokens are under 80% of batch x longest
    sequence (lengths spread widely, or some sequences empty).

    The plan passes this as the library's ragged-lengths hint: larger grids
    then run in smaller workgroups, which balance ragged batches better and
    uniform ones worse. Results agree to FP32 rounding either way.
    """
    lengths = np.asarray(lengths, dtype=np.int64)
    longest = int(lengths.max(initial=0))
    return bool(longest > 0 and int(lengths.sum()) < 0.8 * lengths.size * longest)


def _token_batch(k_new, v_new, layout):
    """Accept [B, Hkv, D] (one token) or [B, tokens, Hkv, D]; returns 4-d views."""
    if k_new.dim() == 3:
        k_new, v_new = k_new.unsqueeze(1), v_new.unsqueeze(1)
    if k_new.dim() != 4 or tuple(k_new.shape) != tuple(v_new.shape) or k_new.shape[0] != layout.batch or \
            tuple(k_new.shape[2:]) != (layout.kv_heads, layout.head_dim) or k_new.shape[1] < 1:
        raise ValueError("new tokens must be [B, Hkv, D] or [B, tokens, Hkv, D] matching the layout")
    return k_new, v_new


_FP8 = (torch.float8_e4m3fn, torch.float8_e5m2)
_STORED = (torch.float32, torch.float16, torch.bfloat16) + _FP8


def _check_formats(q_dtype, k_dtype, v_dtype):
    """q/k/v share float16, bfloat16 or float32, or k/v are FP8 under a 16-bit q."""
    if q_dtype not in (torch.float16, torch.bfloat16, torch.float32) or v_dtype != k_dtype or not (
            k_dtype == q_dtype or (k_dtype in _FP8 and q_dtype != torch.float32)):
        raise TypeError("q/k/v must share float16, bfloat16 or float32 dtype "
                        "(k/v may be float8_e4m3fn/float8_e5m2 with a float16 or bfloat16 q)")


def _check_cache(k_cache, v_cache, k_new, v_new, expected_k, device):
    if tuple(k_cache.shape) != expected_k or tuple(v_cache.shape) != expected_k:
        raise ValueError("cache shape does not match the layout")
    if k_cache.dtype not in _STORED or any(t.dtype != k_cache.dtype for t in (v_cache, k_new, v_new)):
        raise TypeError("cache and new tokens must share one storage dtype "
                        "(float32, float16, bfloat16, float8_e4m3fn or float8_e5m2)")
    for tensor in (k_cache, v_cache, k_new, v_new):
        if tensor.device != device or not tensor.is_contiguous():
            raise ValueError("cache and new tokens must be contiguous on the plan device")


def append_kv(layout: Layout, k_cache, v_cache, table, positions, k_new, v_new):
    """Write new tokens into a paged KV cache at explicit positions.

    ``table`` ``[B, W]`` and ``positions`` ``[B]`` are int32 device tensors;
    token ``j`` of sequence ``b`` goes to logical position
    ``positions[b] + j`` (page ``table[b, pos // T]``, slot ``pos % T``).
    Tokens outside the table's capacity or on page ids outside
    ``[0, physical_pages)`` are skipped. Runs on the current stream.
    """
    expected_k = (layout.physical_pages, layout.page_size, layout.kv_heads, layout.head_dim)
    k_new, v_new = _token_batch(k_new, v_new, layout)
    _check_cache(k_cache, v_cache, k_new, v_new, expected_k, k_cache.device)
    for t in (table, positions):
        if t.device != k_cache.device or t.dtype != torch.int32 or not t.is_contiguous():
            raise TypeError("table and positions must be contiguous int32 tensors on the cache device")
    if table.dim() != 2 or table.shape[0] != layout.batch or tuple(positions.shape) != (layout.batch,):
        raise ValueError("table must be [B, W] and positions [B]")
    load_extension().append_kv(k_new, v_new, table, positions, k_cache, v_cache, False)
