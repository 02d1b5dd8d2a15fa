"""ctypes binding of the C ABI in ``include/paged_decode.h``.

This is the stub an FFI caller (or a maintainer of the reference wiring its
``load_extension`` to this library) would write: plain pointers and ints, the
stream as an opaque pointer. ``PROTOTYPES`` mirrors the header one to one.
"""
import ctypes
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libpaged_decode_hip.so"

# The header's PD_ABI_VERSION these prototypes follow; load() refuses a
# library that reports another (a stale build would read arguments added
# since then, such as length_bounds or max_context, as its stream).
PD_ABI_VERSION = 16

PD_OK = 0
PD_ERR_NULL_POINTER = 1
PD_ERR_SHAPE = 2
PD_ERR_DTYPE = 3
PD_ERR_SPLIT = 4
PD_ERR_MERGE = 5
PD_ERR_LAUNCH = 6
PD_DTYPE_F32 = 0
PD_DTYPE_F16 = 1
PD_DTYPE_BF16 = 2
PD_DTYPE_FP8_E4M3 = 3
PD_DTYPE_FP8_E5M2 = 4
PD_MERGE_SERIAL = 0
PD_MERGE_SHARED = 1
PD_SHARED_MERGE_MAX_PARTS = 4096  # states (4 per split)
PD_HINT_NONE = 0
PD_HINT_UNSHARED_PAGES = 1
PD_HINT_RAGGED_LENGTHS = 2
PD_ERR_HINT = 7
PD_ERR_SCRATCH = 8
PD_ERR_PREFIX = 9
PD_SCRATCH_BYTES = 32 << 20

_P = ctypes.c_void_p
_I = ctypes.c_int
_F = ctypes.c_float


class LaunchPlan(ctypes.Structure):
    """``pd_launch_plan`` of the header."""
    _fields_ = [(name, ctypes.c_uint if name.startswith("grid_") and name != "grid_kind" else ctypes.c_int)
                for name in ("launches", "kernel_splits", "kernel_split_tokens", "grid_x", "grid_y", "grid_z",
                             "waves_per_workgroup", "kv_heads_per_workgroup", "quarters_per_workgroup", "head_tile",
                             "grid_kind", "xcd_grouped", "combined", "stream_mode", "merge_kernel", "merge_loads",
                             "merge_chunk_floats", "merge_xcd_grouped", "merge_state_stride", "shared_prefix_items")]


PROTOTYPES = {
    "pd_decode": (_I, [_P, _P, _P, _I, _P, _P, _P, _P, _P] + [_I] * 10 + [_P]),
    "pd_decode_ex": (_I, [_P, _I, _P, _P, _I, _F, _F, _P, _P, _P, _P, _P] + [_I] * 11 + [_P, _P]),
    "pd_decode_scratch": (_I, [_P, _I, _P, _P, _I, _F, _F, _P, _P, _P] + [_I] * 11 + [_P, _P]),
    "pd_decode_partial": (_I, [_P, _P, _P, _I, _P, _P, _P, _P] + [_I] * 9 + [_P]),
    "pd_decode_partial_ex": (_I, [_P, _I, _P, _P, _I, _F, _F, _P, _P, _P, _P] + [_I] * 10 + [_P, _P]),
    "pd_prefix_runs": (_I, [_P, _I, _I, _P]),
    "pd_decode_prefix": (_I, [_P, _I, _P, _P, _I, _F, _F, _P, _P, _P, _P, _P] + [_I] * 11 + [_P, _P, _P]),
    "pd_decode_partial_prefix": (_I, [_P, _I, _P, _P, _I, _F, _F, _P, _P, _P, _P] + [_I] * 10 + [_P, _P, _P]),
    "pd_decode_merge": (_I, [_P, _P, _P, _P] + [_I] * 8 + [_P]),
    "pd_append_kv": (_I, [_P, _P, _I, _P, _P, _P, _P] + [_I] * 7 + [_P]),
    "pd_append_kv_advance": (_I, [_P, _P, _I, _P, _P, _P, _P] + [_I] * 8 + [_P]),
    "pd_table_from_csr": (_I, [_P, _P, ctypes.c_int64, _P, _P, _P, _P] + [_I] * 4 + [_P]),
    "pd_workspace_bytes": (ctypes.c_size_t, [_I] * 4),
    "pd_decode_launch_count": (_I, [_I] * 12 + [_P]),
    "pd_decode_kernel_split": (_I, [_I] * 11 + [_P, _I, _P, _P]),
    "pd_decode_launch_plan": (_I, [_I] * 13 + [_P, _P, _I, ctypes.POINTER(LaunchPlan)]),
    "pd_stream_read": (_I, [_P, ctypes.c_size_t, _P, ctypes.c_size_t, _P, _P]),
    "pd_status_string": (ctypes.c_char_p, [_I]),
    "pd_abi_version": (_I, []),
}


def load(path=LIBRARY):
    """Load the library and attach the prototypes. Raises OSError if it is
    absent or reports an ABI version other than ``PD_ABI_VERSION``."""
    lib = ctypes.CDLL(str(path))
    lib.pd_abi_version.restype = ctypes.c_int
    lib.pd_abi_version.argtypes = []
    version = lib.pd_abi_version()
    if version != PD_ABI_VERSION:
        raise OSError(f"{path} implements paged_decode ABI {version}, these prototypes follow ABI "
                      f"{PD_ABI_VERSION}: rebuild the library (python -m paged_decode._build)")
    for name, (restype, argtypes) in PROTOTYPES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


def status_string(lib, status):
    return lib.pd_status_string(status).decode()


def launch_count(lib, q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size, table_width,
                 physical_pages, splits, split_tokens, hints=PD_HINT_NONE):
    """Kernel launches of a full decode call of these formats and shapes: 1 (whole
    rows: the partition launch writes the output) or 2 (partition and merge).
    Raises ValueError with the library's message for shapes it rejects."""
    launches = ctypes.c_int(0)
    status = lib.pd_decode_launch_count(q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size,
                                        table_width, physical_pages, splits, split_tokens, hints,
                                        ctypes.byref(launches))
    if status != PD_OK:
        raise ValueError(status_string(lib, status))
    return launches.value


def kernel_split(lib, q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size, table_width,
                 physical_pages, splits, split_tokens, length_bounds=None, compute_units=0):
    """(partitions, tokens per partition) of a full decode call's two launches:
    the caller's (splits, split_tokens), or a coarser split on large grids.
    length_bounds: None or host int32 upper bounds on the lengths [batch].
    Raises ValueError with the library's message for shapes it rejects."""
    import numpy as np

    bounds = None
    if length_bounds is not None:
        bounds = np.ascontiguousarray(length_bounds, dtype=np.int32)
    splits_out, tokens_out = ctypes.c_int(0), ctypes.c_int(0)
    status = lib.pd_decode_kernel_split(q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size,
                                        table_width, physical_pages, splits, split_tokens,
                                        None if bounds is None else bounds.ctypes.data, compute_units,
                                        ctypes.byref(splits_out), ctypes.byref(tokens_out))
    if status != PD_OK:
        raise ValueError(status_string(lib, status))
    return splits_out.value, tokens_out.value


def prefix_runs(lib, table):
    """Shared-prefix runs of a host page table [batch, width] (``pd_prefix_runs``):
    an int32 array [2 * batch] of (leader, leading entries in common with it)."""
    import numpy as np

    table = np.ascontiguousarray(table, dtype=np.int32)
    if table.ndim != 2:
        raise ValueError("table must be [batch, width]")
    runs = np.empty(2 * table.shape[0], dtype=np.int32)
    status = lib.pd_prefix_runs(table.ctypes.data, table.shape[0], table.shape[1], runs.ctypes.data)
    if status != PD_OK:
        raise ValueError(status_string(lib, status))
    return runs


def launch_plan(lib, q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size, table_width,
                physical_pages, splits, split_tokens, merge_mode=PD_MERGE_SERIAL, hints=PD_HINT_NONE,
                length_bounds=None, compute_units=0, prefix_runs=None):
    """The launches of a full decode call (``pd_decode_launch_plan``) as a dict of
    the header's fields. Raises ValueError with the library's message for
    shapes it rejects."""
    import numpy as np

    bounds = None if length_bounds is None else np.ascontiguousarray(length_bounds, dtype=np.int32)
    runs = None if prefix_runs is None else np.ascontiguousarray(prefix_runs, dtype=np.int32)
    plan = LaunchPlan()
    status = lib.pd_decode_launch_plan(q_dtype, kv_dtype, batch, query_heads, kv_heads, head_dim, page_size,
                                       table_width, physical_pages, splits, split_tokens, merge_mode, hints,
                                       None if bounds is None else bounds.ctypes.data,
                                       None if runs is None else runs.ctypes.data, compute_units,
                                       ctypes.byref(plan))
    if status != PD_OK:
        raise ValueError(status_string(lib, status))
    return {name: getattr(plan, name) for name, _ in LaunchPlan._fields_}
