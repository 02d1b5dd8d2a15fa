"""Host-side boundary checks that need no GPU.

* DecodePlan constructor validation (reference runtime.py:33-60): every check
  that precedes the device check raises the reference's exception type.
* The C-ABI library loads, exports every function include/paged_decode.h
  declares, and rejects invalid arguments with the documented status codes
  before touching the GPU.
"""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from gpu_util import no_child_processes_after_gpu_init
from paged_decode import cabi
from paged_decode.layout import Layout
from paged_decode.runtime import DecodePlan

HEADER = Path(__file__).resolve().parent.parent / "include" / "paged_decode.h"


def plan_args():
    return Layout(1, 8, 2, 64, 16, 8), np.arange(8, dtype=np.int32)[None], np.array([127])


@pytest.mark.parametrize("kwargs,exc", [
    (dict(merge="fast"), ValueError),
    (dict(split_tokens=0), ValueError),
    (dict(split_tokens=True), ValueError),
    (dict(split_tokens=2.0), ValueError),
    (dict(split_tokens=np.int64(4)), ValueError),
    (dict(split_tokens=1048577), ValueError),
    (dict(device="cpu"), ValueError),
])
def test_plan_rejects_bad_arguments(kwargs, exc):
    layout, table, lengths = plan_args()
    with pytest.raises(exc):
        DecodePlan(layout, table, lengths, **kwargs)


@pytest.mark.parametrize("max_context", [True, 1.0, 126, 129, -1])
def test_plan_rejects_bad_context_reservation(max_context):
    layout, table, lengths = plan_args()       # lengths [127], table capacity 8 * 16 = 128 tokens
    with pytest.raises(ValueError):
        DecodePlan(layout, table, lengths, max_context=max_context)


@pytest.mark.parametrize("layout", [Layout(1, 8, 2, 96, 16, 8), Layout(1, 8, 2, 64, 8, 8),
                                    Layout(65536, 8, 2, 64, 16, 8), Layout(1, 65536 * 2, 2, 64, 16, 8)])
def test_plan_rejects_unsupported_layouts(layout):
    with pytest.raises(ValueError):
        DecodePlan(layout, np.zeros((layout.batch, 8), dtype=np.int32), np.zeros(layout.batch, dtype=np.int32))


def test_plan_rejects_bad_metadata_and_limits():
    layout = Layout(1, 8, 2, 64, 16, 8)
    with pytest.raises(ValueError):
        DecodePlan(layout, np.array([[0, 9]]), np.array([20]))            # live page out of range
    with pytest.raises(TypeError):
        DecodePlan(layout, np.array([[0., 1.]]), np.array([20]))
    wide = Layout(1, 8, 2, 64, 16, 65537)
    with pytest.raises(ValueError):
        DecodePlan(wide, np.zeros((1, 65537), dtype=np.int32), np.array([1]))  # width > 65536
    long = Layout(1, 8, 2, 64, 32, 40000)
    with pytest.raises(ValueError):
        DecodePlan(long, np.arange(40000, dtype=np.int32)[None], np.array([1048577]))  # > 1M tokens
    with pytest.raises(ValueError):
        DecodePlan(long, np.arange(40000, dtype=np.int32)[None], np.array([70000]), split_tokens=1)


def header_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(pd_\w+)\s*\(", text, re.M)))


def test_header_and_binding_agree():
    assert header_functions() == sorted(cabi.PROTOTYPES)


def test_library_exports_every_declared_symbol():
    lib = cabi.load()
    for name in header_functions():
        assert hasattr(lib, name), name
    assert lib.pd_abi_version() == cabi.PD_ABI_VERSION == 16
    assert re.search(r"#define\s+PD_ABI_VERSION\s+(\d+)", HEADER.read_text()).group(1) == str(cabi.PD_ABI_VERSION)
    assert lib.pd_workspace_bytes(4, 32, 128, 16) == 4_259_840  # reference docs/DESIGN.md:76
    assert lib.pd_workspace_bytes(0, 32, 128, 16) == 0
    assert "success" in cabi.status_string(lib, cabi.PD_OK)
    assert cabi.status_string(lib, 99) == "unknown status"


def test_ctypes_binding_refuses_another_abi_version(monkeypatch):
    """cabi.load compares pd_abi_version() with the version its prototypes
    follow before attaching them: against a library of another ABI the
    widened entries would read their new arguments as the stream."""
    monkeypatch.setattr(cabi, "PD_ABI_VERSION", cabi.PD_ABI_VERSION - 1)
    with pytest.raises(OSError, match="ABI"):
        cabi.load()


def test_launch_count_query():
    """Whole-row launches (one kernel) for rows of at most 128 KB of K and V per
    (sequence, KV head); partition + merge otherwise; shape errors as pd_decode_ex."""
    lib = cabi.load()
    f32, f16, fp8 = cabi.PD_DTYPE_F32, cabi.PD_DTYPE_F16, cabi.PD_DTYPE_FP8_E4M3
    # FP32 oracle case: B2, 8/2 heads, D64, page 16, 16 pages per row, split 256 (256 tokens: 128 KB).
    assert cabi.launch_count(lib, f32, f32, 2, 8, 2, 64, 16, 16, 32, 1, 256) == 1
    # Llama-3-8B decode shape (4096 tokens per row) and MQA B128 L1024 D64 (256 KB per row).
    assert cabi.launch_count(lib, f16, f16, 4, 32, 8, 128, 16, 256, 1024, 16, 256) == 2
    assert cabi.launch_count(lib, f16, f16, 128, 16, 1, 64, 16, 64, 8192, 4, 256) == 2
    # The bound is on splits * split_tokens, capped by the table: 512 FP16 tokens at D128 is 256 KB,
    # 512 FP8 tokens 128 KB; a 4096-token reservation in a 256-token table still fits.
    assert cabi.launch_count(lib, f16, f16, 8, 32, 8, 128, 16, 32, 256, 2, 256) == 2
    assert cabi.launch_count(lib, f16, fp8, 8, 32, 8, 128, 16, 32, 256, 2, 256) == 1
    assert cabi.launch_count(lib, f16, f16, 8, 32, 8, 64, 16, 16, 128, 16, 256) == 1
    with pytest.raises(ValueError, match="dimension"):
        cabi.launch_count(lib, f16, f16, 8, 32, 8, 96, 16, 16, 128, 1, 256)
    with pytest.raises(ValueError, match="dtype"):
        cabi.launch_count(lib, f32, fp8, 8, 32, 8, 64, 16, 16, 128, 1, 256)



def test_kernel_split_query():
    """Full calls on grids of many waves per CU run over coarser partitions (a
    power of two times split_tokens, at most 128 KB of K and V per wave, at
    least 8 waves per CU); single-round grids, whole-row calls and FP32 keep
    the caller's split."""
    from paged_decode.workload import make_workload

    lib = cabi.load()
    f32, f16, fp8 = cabi.PD_DTYPE_F32, cabi.PD_DTYPE_F16, cabi.PD_DTYPE_FP8_E4M3

    def split(q, kv, b, hq, hkv, d, t, w, p, s, st, bounds=None, cus=256):
        return cabi.kernel_split(lib, q, kv, b, hq, hkv, d, t, w, p, s, st, bounds, cus)

    # Llama-3-8B B4 L4096 (FP16 and FP8 K/V) and MQA B128 L1024: eight waves per CU at most, kept.
    assert split(f16, f16, 4, 32, 8, 128, 16, 256, 1024, 16, 256, [4096] * 4) == (16, 256)
    assert split(f16, fp8, 4, 32, 8, 128, 16, 256, 1024, 16, 256, [4096] * 4) == (16, 256)
    assert split(f16, f16, 128, 16, 1, 64, 16, 64, 8192, 4, 256, [1024] * 128) == (4, 256)
    # Uniform B16 L4096: 32 waves per CU at split 256; 128 KB per wave caps it at 1024 tokens.
    assert split(f16, f16, 16, 32, 8, 128, 16, 256, 4096, 16, 256, [4096] * 16) == (4, 1024)
    # FP8 K/V and D64 MQA reach 1024 tokens at 64 KB per wave, where eight waves per CU remain.
    assert split(f16, fp8, 16, 32, 8, 128, 16, 256, 4096, 16, 256, [4096] * 16) == (4, 1024)
    assert split(f16, f16, 512, 16, 1, 64, 16, 64, 32768, 4, 256, [1024] * 512) == (1, 1024)
    # 32K-context MHA at split 128: 128 waves per CU -> 1024-token partitions.
    assert split(f16, f16, 1, 32, 32, 128, 16, 2048, 2048, 256, 128, [32768]) == (32, 1024)
    # The ragged + shared-prefix batch at split 128 (host lengths as bounds): 512-token partitions.
    w = make_workload("ragged_shared_b16")
    lay = w.layout
    splits = -(-int(w.lengths.max()) // 128)
    assert split(f16, f16, lay.batch, lay.query_heads, lay.kv_heads, lay.head_dim, lay.page_size, w.table.shape[1],
                 lay.physical_pages, splits, 128, w.lengths) == (-(-splits // 4), 512)
    # Bounds that reach few partitions keep the split, and so does a call without bounds.
    assert split(f16, f16, 16, 32, 8, 128, 16, 256, 4096, 16, 256, [0] * 16) == (16, 256)
    assert split(f16, f16, 16, 32, 8, 128, 16, 256, 4096, 16, 256) == (16, 256)
    # Twice the CUs need twice the waves.
    assert split(f16, f16, 16, 32, 8, 128, 16, 256, 4096, 16, 256, [4096] * 16, cus=512) == (8, 512)
    # FP32 inputs and whole-row calls keep the caller's split.
    assert split(f32, f32, 16, 32, 8, 128, 16, 256, 4096, 16, 256, [4096] * 16) == (16, 256)
    assert split(f16, f16, 4096, 32, 8, 64, 16, 8, 32768, 2, 64, [128] * 4096) == (2, 64)
    # Whatever the rule picks, fewer partitions cover at least the caller's tokens.
    rng = np.random.default_rng(5)
    for _ in range(200):
        b, hkv = int(rng.integers(1, 65)), int(rng.choice([1, 2, 4, 8, 32]))
        hq = hkv * int(rng.choice([1, 4, 8, 16]))
        d, t = int(rng.choice([64, 128])), int(rng.choice([16, 32]))
        width = int(rng.integers(1, 513))
        st = int(rng.choice([16, 64, 128, 256, 512, 1000]))
        s = max(1, -(-width * t // st))
        kv = int(rng.choice([f16, fp8]))
        bounds = rng.integers(0, width * t + 1, size=b) if rng.random() < 0.5 else None
        ks, kst = split(f16, kv, b, hq, hkv, d, t, width, b * width, s, st, bounds)
        c = kst // st
        assert kst % st == 0 and c & (c - 1) == 0 and ks == -(-s // c) and ks * kst >= s * st
        assert c == 1 or (kst // 4) * d * (1 if kv == fp8 else 2) * 2 <= 128 * 1024
    with pytest.raises(ValueError, match="dimension"):
        split(f16, f16, 8, 32, 8, 96, 16, 16, 128, 1, 256)


C_CONSUMER = r"""
#include <stdio.h>
#include <string.h>
#include "paged_decode.h"

int main(void) {
    if (pd_abi_version() != PD_ABI_VERSION || PD_ABI_VERSION != 16) return 1;
    if (pd_workspace_bytes(4, 32, 128, 16) != 4259840u) return 2;
    /* Rejected before any launch: no device is touched. */
    if (pd_decode(NULL, NULL, NULL, PD_DTYPE_F16, NULL, NULL, NULL, NULL, NULL,
                  4, 32, 8, 128, 16, 256, 1024, 16, 256, PD_MERGE_SERIAL, NULL) != PD_ERR_NULL_POINTER) return 3;
    if (pd_append_kv(NULL, NULL, PD_DTYPE_FP8_E4M3, NULL, NULL, NULL, NULL,
                     4, 1, 8, 128, 16, 256, 1024, NULL) != PD_ERR_NULL_POINTER) return 4;
    if (strstr(pd_status_string(PD_ERR_SHAPE), "dimension") == NULL) return 5;
    if (pd_table_from_csr(NULL, NULL, 0, NULL, NULL, NULL, NULL, 4, 256, 16, 4096, NULL) != PD_ERR_NULL_POINTER) return 6;
    if (strstr(pd_status_string(PD_ERR_HINT), "hint") == NULL || PD_HINT_UNSHARED_PAGES != 1 ||
        PD_HINT_RAGGED_LENGTHS != 2) return 7;
    if (pd_stream_read(NULL, 16, NULL, 0, NULL, NULL) != PD_ERR_NULL_POINTER) return 8;
    puts("ok");
    return 0;
}
"""


def test_header_is_plain_c_and_library_links_from_c(tmp_path):
    """A C99 FFI consumer: compiles against the header with gcc, links and runs (no GPU call)."""
    import shutil
    import subprocess

    no_child_processes_after_gpu_init()
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    src = tmp_path / "consumer.c"
    src.write_text(C_CONSUMER)
    exe = tmp_path / "consumer"
    libdir = cabi.LIBRARY.parent
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-pedantic", f"-I{HEADER.parent}", str(src),
                    f"-L{libdir}", "-lpaged_decode_hip", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert run.returncode == 0 and run.stdout.strip() == "ok", (run.returncode, run.stdout, run.stderr)


def test_extension_exports_reference_entry():
    from paged_decode.runtime import load_extension

    ext = load_extension()
    for name in ("decode", "partial", "merge", "append_kv", "table_from_csr", "workspace_bytes", "abi_version"):
        assert hasattr(ext, name)
    assert ext.workspace_bytes(4, 32, 128, 16) == 4_259_840


def fake(n=1):
    """Distinct non-null host addresses; validation rejects before any use."""
    buf = (ctypes.c_char * (64 * n))()
    return [ctypes.addressof(buf) + 64 * i for i in range(n)], buf


BASE = dict(dtype=1, batch=4, query_heads=32, kv_heads=8, head_dim=128, page_size=16, table_width=256,
            physical_pages=1024, splits=16, split_tokens=256, merge_mode=0)


def call_decode(lib, ptrs, **over):
    a = {**BASE, **over}
    return lib.pd_decode(ptrs[0], ptrs[1], ptrs[2], a["dtype"], ptrs[3], ptrs[4], ptrs[5], ptrs[6], ptrs[7],
                         a["batch"], a["query_heads"], a["kv_heads"], a["head_dim"], a["page_size"],
                         a["table_width"], a["physical_pages"], a["splits"], a["split_tokens"],
                         a["merge_mode"], None)


@pytest.mark.parametrize("over,status", [
    (dict(dtype=7), cabi.PD_ERR_DTYPE),
    (dict(dtype=cabi.PD_DTYPE_FP8_E4M3), cabi.PD_ERR_DTYPE),   # FP8 q is not a supported pair
    (dict(batch=0), cabi.PD_ERR_SHAPE),
    (dict(batch=65536), cabi.PD_ERR_SHAPE),
    (dict(query_heads=30), cabi.PD_ERR_SHAPE),
    (dict(head_dim=96), cabi.PD_ERR_SHAPE),
    (dict(page_size=8), cabi.PD_ERR_SHAPE),
    (dict(table_width=65537), cabi.PD_ERR_SHAPE),
    (dict(physical_pages=0), cabi.PD_ERR_SHAPE),
    (dict(splits=0), cabi.PD_ERR_SPLIT),
    (dict(splits=65536), cabi.PD_ERR_SPLIT),
    (dict(split_tokens=0), cabi.PD_ERR_SPLIT),
    (dict(split_tokens=(1 << 20) + 1), cabi.PD_ERR_SPLIT),
    (dict(merge_mode=2), cabi.PD_ERR_MERGE),
    (dict(merge_mode=1, splits=1025), cabi.PD_ERR_MERGE),
])
def test_c_abi_rejects_invalid_arguments(over, status):
    lib = cabi.load()
    ptrs, _keep = fake(8)
    assert call_decode(lib, ptrs, **over) == status


def test_c_abi_rejects_null_pointers():
    lib = cabi.load()
    ptrs, _keep = fake(8)
    for i in range(8):
        broken = list(ptrs)
        broken[i] = None
        assert call_decode(lib, broken) == cabi.PD_ERR_NULL_POINTER
    merge_args = dict(batch=4, query_heads=32, head_dim=128, page_size=16, table_width=256, splits=16,
                      split_tokens=256)

    def call_merge(num, st, out, lengths, merge_mode=0, **over):
        a = {**merge_args, **over}
        return lib.pd_decode_merge(num, st, out, lengths, a["batch"], a["query_heads"], a["head_dim"],
                                   a["page_size"], a["table_width"], a["splits"], a["split_tokens"], merge_mode,
                                   None)

    assert call_merge(None, ptrs[1], ptrs[2], ptrs[3]) == cabi.PD_ERR_NULL_POINTER
    assert call_merge(ptrs[0], ptrs[1], ptrs[2], None) == cabi.PD_ERR_NULL_POINTER
    assert call_merge(ptrs[0], ptrs[1], ptrs[2], ptrs[3], merge_mode=7) == cabi.PD_ERR_MERGE
    assert call_merge(ptrs[0], ptrs[1], ptrs[2], ptrs[3], page_size=8) == cabi.PD_ERR_SHAPE
    assert call_merge(ptrs[0], ptrs[1], ptrs[2], ptrs[3], split_tokens=0) == cabi.PD_ERR_SPLIT
    assert lib.pd_decode_partial(ptrs[0], ptrs[1], ptrs[2], 1, ptrs[3], ptrs[4], ptrs[5], ptrs[6],
                                 4, 32, 8, 128, 16, 256, 1024, 0, 256, None) == cabi.PD_ERR_SPLIT


def test_append_entries_reject_invalid_arguments():
    lib = cabi.load()
    ptrs, _keep = fake(8)
    base = dict(dtype=1, batch=4, tokens=1, kv_heads=8, head_dim=128, page_size=16, table_width=256,
                physical_pages=1024)

    def call(fn, ptr_over=None, max_context=None, **over):
        a = {**base, **over}
        p = list(ptrs)
        for i, value in (ptr_over or {}).items():
            p[i] = value
        args = [p[0], p[1], a["dtype"], p[2], p[3], p[4], p[5], a["batch"], a["tokens"], a["kv_heads"],
                a["head_dim"], a["page_size"], a["table_width"], a["physical_pages"]]
        if fn is lib.pd_append_kv_advance:
            args.append(4096 if max_context is None else max_context)
        return fn(*args, None)

    for fn in (lib.pd_append_kv, lib.pd_append_kv_advance):
        for i in range(6):
            assert call(fn, {i: None}) == cabi.PD_ERR_NULL_POINTER
        assert call(fn, dtype=5) == cabi.PD_ERR_DTYPE
        for over in (dict(batch=0), dict(tokens=0), dict(head_dim=96), dict(page_size=8), dict(table_width=0),
                     dict(physical_pages=0)):
            assert call(fn, **over) == cabi.PD_ERR_SHAPE
    # The advance entry's context capacity: 0 .. 1048576 tokens.
    for max_context in (-1, (1 << 20) + 1):
        assert call(lib.pd_append_kv_advance, max_context=max_context) == cabi.PD_ERR_SHAPE


@pytest.mark.parametrize("q_dtype,kv_dtype,k_scale,v_scale", [
    (cabi.PD_DTYPE_F32, cabi.PD_DTYPE_FP8_E4M3, 1.0, 1.0),   # FP8 K/V need a 16-bit q
    (cabi.PD_DTYPE_F16, cabi.PD_DTYPE_BF16, 1.0, 1.0),       # mixed 16-bit formats
    (cabi.PD_DTYPE_BF16, cabi.PD_DTYPE_F32, 1.0, 1.0),
    (cabi.PD_DTYPE_F16, cabi.PD_DTYPE_FP8_E5M2, 0.0, 1.0),   # scales must be > 0 and finite
    (cabi.PD_DTYPE_F16, cabi.PD_DTYPE_FP8_E5M2, 1.0, float("nan")),
    (cabi.PD_DTYPE_F16, cabi.PD_DTYPE_FP8_E4M3, float("inf"), 1.0),
])
def test_extended_entry_rejects_formats_and_scales(q_dtype, kv_dtype, k_scale, v_scale):
    lib = cabi.load()
    ptrs, _keep = fake(8)
    status = lib.pd_decode_ex(ptrs[0], q_dtype, ptrs[1], ptrs[2], kv_dtype, k_scale, v_scale, ptrs[3], ptrs[4],
                              ptrs[5], ptrs[6], ptrs[7], 4, 32, 8, 128, 16, 256, 1024, 16, 256, 0, 0, None, None)
    assert status == cabi.PD_ERR_DTYPE
    status = lib.pd_decode_partial_ex(ptrs[0], q_dtype, ptrs[1], ptrs[2], kv_dtype, k_scale, v_scale, ptrs[3],
                                      ptrs[4], ptrs[5], ptrs[6], 4, 32, 8, 128, 16, 256, 1024, 16, 256, 0, None, None)
    assert status == cabi.PD_ERR_DTYPE


@pytest.mark.parametrize("hints", [4, 8, 7, -1, 1 << 30])
def test_extended_entries_reject_unknown_hints(hints):
    """Only PD_HINT_UNSHARED_PAGES and PD_HINT_RAGGED_LENGTHS are defined; other bits are rejected before
    any launch."""
    lib = cabi.load()
    ptrs, _keep = fake(8)
    f16 = cabi.PD_DTYPE_F16
    status = lib.pd_decode_ex(ptrs[0], f16, ptrs[1], ptrs[2], f16, 1.0, 1.0, ptrs[3], ptrs[4], ptrs[5], ptrs[6],
                              ptrs[7], 4, 32, 8, 128, 16, 256, 1024, 16, 256, 0, hints, None, None)
    assert status == cabi.PD_ERR_HINT
    status = lib.pd_decode_partial_ex(ptrs[0], f16, ptrs[1], ptrs[2], f16, 1.0, 1.0, ptrs[3], ptrs[4], ptrs[5],
                                      ptrs[6], 4, 32, 8, 128, 16, 256, 1024, 16, 256, hints, None, None)
    assert status == cabi.PD_ERR_HINT
    assert "hint" in cabi.status_string(lib, cabi.PD_ERR_HINT)


def test_ragged_lengths_hint_follows_the_lengths():
    """The plan's ragged-lengths hint: live tokens under 80% of batch x longest."""
    from paged_decode.runtime import ragged_lengths

    assert not ragged_lengths(np.array([4096, 4096, 4096, 4096]))
    assert not ragged_lengths(np.array([0, 0]))                      # no tokens at all
    assert not ragged_lengths(np.array([100, 90, 85, 80]))           # 355 of 400: 89%
    assert ragged_lengths(np.array([100, 60, 60, 60]))               # 280 of 400: 70%
    assert ragged_lengths(np.array([4096, 0]))
    assert not ragged_lengths(np.array([5, 4, 4, 4, 4]))             # 21 of 25: exactly 84%
    assert not ragged_lengths(np.array([5, 4, 4, 4, 3]))             # 20 of 25: 80%, not under it
    assert ragged_lengths(np.array([5, 4, 4, 4, 2]))                 # 19 of 25: 76%
    assert not ragged_lengths(np.array([5, 4, 4, 4, 3])[:4])         # 17 of 20: 85%


def test_page_sharing_hint_follows_the_table():
    """unshared_pages: any page id mapped twice among the entries up to the
    reserved capacity (padding excluded) means shared."""
    from paged_decode.runtime import unshared_pages

    table = np.array([[0, 1, 2, -1], [3, 4, -1, -1]], dtype=np.int32)
    assert unshared_pages(table, 16, 64)
    prefix = np.array([[0, 1, 2, -1], [0, 4, -1, -1]], dtype=np.int32)      # page 0 in both rows
    assert not unshared_pages(prefix, 16, 64)
    late = np.array([[0, 1, 2, 5], [3, 4, -1, 5]], dtype=np.int32)          # page 5 aliased in the last column
    assert not unshared_pages(late, 16, 64)
    assert unshared_pages(late, 16, 48)                                      # beyond the reserved capacity
    within = np.array([[7, 7, -1, -1], [3, -1, -1, -1]], dtype=np.int32)    # twice within one sequence
    assert not unshared_pages(within, 16, 64)


def test_table_from_csr_rejects_invalid_arguments():
    """pd_table_from_csr: null pointers (overflow may be NULL; indices too when it holds no entry) and
    dimensions, before any launch."""
    lib = cabi.load()
    ptrs, _keep = fake(6)

    def call(indptr, indices, last, table, lengths, overflow, batch=4, width=256, page=16, max_context=4096,
             count=100):
        return lib.pd_table_from_csr(indptr, indices, count, last, table, lengths, overflow, batch, width, page,
                                     max_context, None)

    for i in range(5):
        broken = list(ptrs[:5])
        broken[i] = None
        assert call(*broken, ptrs[5]) == cabi.PD_ERR_NULL_POINTER
    for over in (dict(batch=0), dict(batch=65536), dict(width=0), dict(width=65537), dict(page=8),
                 dict(max_context=-1), dict(max_context=(1 << 20) + 1), dict(count=-1)):
        assert call(*ptrs, **over) == cabi.PD_ERR_SHAPE, over


def test_scratch_entry_rejects_before_touching_a_device():
    """pd_decode_scratch checks pointers, shapes and the PD_SCRATCH_BYTES bound on the host, before any
    runtime call (no GPU here)."""
    lib = cabi.load()
    ptrs, _keep = fake(6)
    f16 = cabi.PD_DTYPE_F16

    def call(out=ptrs[5], batch=4, heads=32, splits=16, merge=0, hints=0):
        return lib.pd_decode_scratch(ptrs[0], f16, ptrs[1], ptrs[2], f16, 1.0, 1.0, ptrs[3], ptrs[4], out, batch,
                                     heads, 8, 128, 16, 256, 1024, splits, 256, merge, hints, None, None)

    assert call(out=None) == cabi.PD_ERR_NULL_POINTER
    assert call(batch=0) == cabi.PD_ERR_SHAPE
    assert call(merge=3) == cabi.PD_ERR_MERGE
    assert call(hints=4) == cabi.PD_ERR_HINT
    # 64 x 64 rows of 4 x 64 states of 520 bytes: 545 MB of states, far above the 32 MiB scratch.
    assert call(batch=64, heads=64, splits=64) == cabi.PD_ERR_SCRATCH
    # B1 Hq32 D128 takes 32 * 4 * 520 B = 66,560 B of states per split: 504 splits fit, 505 do not.
    assert call(batch=1, heads=32, splits=505) == cabi.PD_ERR_SCRATCH
    assert "scratch" in cabi.status_string(lib, cabi.PD_ERR_SCRATCH)
    assert cabi.PD_SCRATCH_BYTES == 32 << 20


# ---------------------------------------------------------------------------
# No child process after GPU initialisation. A program started from a process
# that has initialised the GPU can take the GPU runtime down with it, so every
# path that would start one (a compiler for a missing build, make for the C
# restatement, git for the build record) refuses or skips instead. The GPU
# state is simulated by patching torch.cuda.is_initialized.


@pytest.fixture
def gpu_initialised(monkeypatch):
    import torch

    monkeypatch.setattr(torch.cuda, "is_initialized", lambda: True)


def test_missing_build_is_refused_after_gpu_init(gpu_initialised, monkeypatch):
    from paged_decode import _build, runtime

    def no_build(*args, **kwargs):
        raise AssertionError("a build was started")

    monkeypatch.setattr(_build, "built", lambda: False)
    monkeypatch.setattr(_build, "build", no_build)
    runtime.load_extension.cache_clear()
    try:
        with pytest.raises(RuntimeError, match="child process"):
            runtime.load_extension()
    finally:
        runtime.load_extension.cache_clear()


def test_compiler_runs_are_refused_after_gpu_init(gpu_initialised):
    from paged_decode import _build

    with pytest.raises(RuntimeError, match="child process"):
        _build._run(["hipcc", "--version"], verbose=False)
    assert _build.git_dirty() is None  # no git process either


def test_oracle_build_is_refused_after_gpu_init(gpu_initialised):
    from oracle import cpu

    with pytest.raises(RuntimeError, match="GPU"):
        cpu.build()


def test_spawning_cpu_tests_skip_after_gpu_init(gpu_initialised):
    with pytest.raises(pytest.skip.Exception):
        no_child_processes_after_gpu_init()


def test_stream_read_rejects_bad_arguments_before_any_launch():
    """pd_stream_read checks pointers and 16-byte granularity on the host."""
    lib = cabi.load()
    ptrs, _keep = fake(3)
    assert lib.pd_stream_read(ptrs[0], 32, ptrs[1], 32, None, None) == cabi.PD_ERR_NULL_POINTER
    assert lib.pd_stream_read(None, 32, ptrs[1], 32, ptrs[2], None) == cabi.PD_ERR_NULL_POINTER
    assert lib.pd_stream_read(ptrs[0], 24, ptrs[1], 32, ptrs[2], None) == cabi.PD_ERR_SHAPE
    assert lib.pd_stream_read(ptrs[0] + 8, 32, ptrs[1], 32, ptrs[2], None) == cabi.PD_ERR_SHAPE
    assert lib.pd_stream_read(None, 0, None, 0, ptrs[2], None) == cabi.PD_OK  # nothing to read: no launch


def test_launch_plan_query_agrees_with_the_other_queries():
    """pd_decode_launch_plan describes the launches pd_decode_ex makes: its launch
    count and kernel split equal pd_decode_launch_count's and
    pd_decode_kernel_split's, and the Llama-3-8B shape with host bounds on 256
    CUs is the XCD-grouped mid-size grid (2 KV heads x 2 quarters per 4-wave
    workgroup, 512 workgroups) merged by XCD-grouped column chunks."""
    lib = cabi.load()
    f32, f16, fp8 = cabi.PD_DTYPE_F32, cabi.PD_DTYPE_F16, cabi.PD_DTYPE_FP8_E4M3
    cases = [(f16, f16, 4, 32, 8, 128, 16, 256, 1024, 16, 256, [4096] * 4),
             (f16, f16, 4, 32, 8, 128, 16, 256, 1024, 16, 256, None),
             (f16, fp8, 128, 16, 1, 64, 16, 64, 8192, 4, 256, [1024] * 128),
             (f32, f32, 2, 8, 2, 64, 16, 16, 32, 1, 256, [100, 256]),
             (f16, f16, 16, 32, 8, 128, 32, 256, 4096, 64, 128, list(range(0, 8192, 512)))]
    for q, kv, b, hq, hkv, d, t, w, p, s, st, bounds in cases:
        plan = cabi.launch_plan(lib, q, kv, b, hq, hkv, d, t, w, p, s, st, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_NONE,
                                bounds, 256)
        assert plan["launches"] == cabi.launch_count(lib, q, kv, b, hq, hkv, d, t, w, p, s, st)
        assert (plan["kernel_splits"], plan["kernel_split_tokens"]) == cabi.kernel_split(
            lib, q, kv, b, hq, hkv, d, t, w, p, s, st, bounds, 256)
        assert (plan["merge_kernel"] == -1) == (plan["launches"] == 1)
        assert plan["grid_x"] * plan["grid_y"] * plan["grid_z"] >= 1 and 1 <= plan["waves_per_workgroup"] <= 16
    llama = cabi.launch_plan(lib, f16, f16, 4, 32, 8, 128, 16, 256, 1024, 16, 256, cabi.PD_MERGE_SERIAL,
                             cabi.PD_HINT_UNSHARED_PAGES, [4096] * 4, 256)
    assert llama["xcd_grouped"] == 1 and llama["kv_heads_per_workgroup"] == 2 and llama["quarters_per_workgroup"] == 2
    assert llama["waves_per_workgroup"] == 4 and llama["grid_x"] * llama["grid_y"] * llama["grid_z"] == 512
    assert llama["merge_kernel"] == 1 and llama["merge_xcd_grouped"] == 1 and llama["merge_chunk_floats"] == 32
    with pytest.raises(ValueError):
        cabi.launch_plan(lib, f16, f16, 4, 32, 8, 96, 16, 256, 1024, 16, 256)


def test_prefix_runs_of_a_host_table():
    """pd_prefix_runs: each sequence's leader is the first sequence whose row
    starts with the same page (-1 when its first entry is not a page) and its
    run the leading entries it has in common with the leader's row, up to the
    first difference or negative entry. A hand-worked table, then random tables
    with shared prefixes against a brute-force longest common prefix."""
    lib = cabi.load()
    table = np.array([[5, 6, 7, 8], [5, 6, 9, 10], [1, 2, 3, 4], [5, 6, 7, -1], [-1, -1, -1, -1], [1, 2, 3, 0],
                      [5, 6, 7, 8]], dtype=np.int32)
    assert cabi.prefix_runs(lib, table).tolist() == [0, 4, 0, 2, 2, 4, 0, 3, -1, 0, 2, 3, 0, 4]
    rng = np.random.default_rng(5)
    for _ in range(50):
        batch, width = int(rng.integers(1, 20)), int(rng.integers(1, 40))
        table = rng.integers(-1, 6, size=(batch, width)).astype(np.int32)
        for b in range(1, batch):  # some rows copy a prefix of an earlier one
            if rng.random() < 0.6:
                src, n = int(rng.integers(0, b)), int(rng.integers(0, width + 1))
                table[b, :n] = table[src, :n]
        runs = cabi.prefix_runs(lib, table)
        for b in range(batch):
            leader, run = int(runs[2 * b]), int(runs[2 * b + 1])
            if table[b, 0] < 0:
                assert (leader, run) == (-1, 0)
                continue
            assert leader == next(c for c in range(b + 1) if table[c, 0] == table[b, 0])
            lcp = 0
            while lcp < width and table[b, lcp] >= 0 and table[b, lcp] == table[leader, lcp]:
                lcp += 1
            assert run == lcp


def test_shared_prefix_items_in_the_launch_plan():
    """With prefix runs and host bounds, the work list of the ragged + shared
    prefix workload scores its shared partitions for several sequences at once
    (fewer workgroups, shared_prefix_items > 0). Without bounds, with FP32
    inputs or with unshared rows there are none; malformed runs are refused
    with PD_ERR_PREFIX."""
    from paged_decode.workload import make_workload

    lib = cabi.load()
    w = make_workload("ragged_shared_b16")
    L = w.layout
    runs = cabi.prefix_runs(lib, w.table)
    splits = -(-int(w.lengths.max()) // w.split_tokens)
    shape = (L.batch, L.query_heads, L.kv_heads, L.head_dim, L.page_size, w.table.shape[1], L.physical_pages, splits,
             w.split_tokens)
    f16, f32 = cabi.PD_DTYPE_F16, cabi.PD_DTYPE_F32
    args = (cabi.PD_MERGE_SERIAL, cabi.PD_HINT_RAGGED_LENGTHS, w.lengths)
    grouped = cabi.launch_plan(lib, f16, f16, *shape, *args, 256, runs)
    plain = cabi.launch_plan(lib, f16, f16, *shape, *args, 256)
    assert plain["shared_prefix_items"] == 0 and plain["grid_kind"] == 2
    assert 0 < grouped["shared_prefix_items"] <= 128 and grouped["grid_kind"] == 2
    assert grouped["grid_x"] < plain["grid_x"] and grouped["kernel_split_tokens"] == plain["kernel_split_tokens"]
    assert cabi.launch_plan(lib, f16, f16, *shape, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_RAGGED_LENGTHS, None, 256,
                            runs)["shared_prefix_items"] == 0
    assert cabi.launch_plan(lib, f32, f32, *shape, *args, 256, runs)["shared_prefix_items"] == 0
    private = np.array([[b, 0] for b in range(L.batch)], dtype=np.int32).reshape(-1)
    assert cabi.launch_plan(lib, f16, f16, *shape, *args, 256, private)["shared_prefix_items"] == 0
    for bad in ([L.batch, 1], [-2, 1], [0, w.table.shape[1] + 1], [0, -1]):
        broken = runs.copy()
        broken[2:4] = bad
        with pytest.raises(ValueError, match="shared-prefix runs"):
            cabi.launch_plan(lib, f16, f16, *shape, *args, 256, broken)


def _sample_table(batch, width, shared):
    """Page table of `batch` samples of one prompt: the first `shared`
    entries of every row are sequence 0's, the rest pages of their own."""
    table = np.zeros((batch, width), dtype=np.int32)
    table[0] = np.arange(width)
    nxt = width
    for b in range(1, batch):
        table[b, :shared] = table[0, :shared]
        table[b, shared:] = np.arange(nxt, nxt + width - shared)
        nxt += width - shared
    return table, nxt


@pytest.mark.parametrize("batch,context,shared_share,finer", [
    (16, 4096, 2, True),    # half the prompt shared: items over 512-token partitions
    (8, 8192, 2, True),
    (32, 2048, 2, True),
    (16, 4096, 4, False),   # a quarter shared: items would save too little, 1024 tokens stay
])
def test_shared_prompt_samples_take_half_the_coarse_split(batch, context, shared_share, finer):
    """Equal-length samples of one prompt (8 KV heads, GQA 4, page 16,
    split 256, 256 CUs): without runs the full call runs over 1024-token
    partitions; with runs, where grouping over 512-token partitions saves at
    least a quarter of them and still fills the device, it runs over 512 with
    shared-prefix items, else it keeps 1024."""
    lib = cabi.load()
    width = context // 16
    table, pages = _sample_table(batch, width, width // shared_share)
    runs = cabi.prefix_runs(lib, table)
    lengths = np.full(batch, context, dtype=np.int32)
    shape = (batch, 32, 8, 128, 16, width, pages, context // 256, 256)
    f16 = cabi.PD_DTYPE_F16
    plain = cabi.launch_plan(lib, f16, f16, *shape, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_NONE, lengths, 256)
    grouped = cabi.launch_plan(lib, f16, f16, *shape, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_NONE, lengths, 256, runs)
    assert plain["kernel_split_tokens"] == 1024 and plain["shared_prefix_items"] == 0
    assert cabi.kernel_split(lib, f16, f16, *shape, lengths, 256) == (context // 1024, 1024)
    if finer:
        assert grouped["kernel_split_tokens"] == 512 and grouped["kernel_splits"] == context // 512
        assert grouped["shared_prefix_items"] > 0 and grouped["grid_kind"] == 2
    else:
        assert grouped["kernel_split_tokens"] == 1024 and grouped["shared_prefix_items"] == 0


def test_launch_planner_invariants_over_random_shapes():
    """The launch planner (`pd_decode_launch_plan`, host only) over 3000 seeded
    random calls: formats, head layouts, pages, table widths up to 4096,
    splits from 1 to the whole context, batches up to 2048, no / exact / low
    / zero / excess host bounds, and prefix runs from tables with and without
    shared prefixes. Every call is planned (or refused with ValueError for a
    shape the checks reject), and the plan keeps the limits the launches rely
    on: a kernel split that is the caller's times a power of two with no more
    partitions than the caller's, grid dimensions the hardware takes,
    workgroups of at most 1024 threads, at most 128 shared-prefix items and
    none without runs and bounds or for FP32 inputs, and the caller's split
    for FP32 inputs."""
    lib = cabi.load()
    rng = np.random.default_rng(8642)
    formats = [(cabi.PD_DTYPE_F16, cabi.PD_DTYPE_F16), (cabi.PD_DTYPE_BF16, cabi.PD_DTYPE_BF16),
               (cabi.PD_DTYPE_F32, cabi.PD_DTYPE_F32), (cabi.PD_DTYPE_F16, cabi.PD_DTYPE_FP8_E4M3),
               (cabi.PD_DTYPE_BF16, cabi.PD_DTYPE_FP8_E5M2)]
    planned = grouped = 0
    for case in range(3000):
        q_dtype, kv_dtype = formats[int(rng.integers(0, len(formats)))]
        kv = int(rng.choice([1, 2, 3, 4, 5, 8, 12, 16, 32]))
        group = int(rng.choice([1, 2, 3, 4, 8, 16, 24, 32]))
        dim = int(rng.choice([64, 128]))
        page = int(rng.choice([16, 32]))
        batch = int(rng.choice([1, 2, 3, 4, 8, 16, 33, 64, 65, 128, 512, 2048]))
        width = int(rng.choice([1, 2, 7, 16, 64, 256, 1024, 4096]))
        if batch * width > 1 << 20:
            width = max(1, (1 << 20) // batch)
        capacity = width * page
        split = int(rng.choice([16, 32, 64, 100, 128, 256, 512, 1024, 4096]))
        splits = max(1, -(-int(rng.integers(1, capacity + 1)) // split))
        lengths = rng.integers(0, min(capacity, splits * split) + 1, batch).astype(np.int32)
        bounds_kind = int(rng.integers(0, 5))
        bounds = [None, lengths, lengths // 2, np.zeros_like(lengths), lengths + 100][bounds_kind]
        runs = None
        if batch <= 128 and width <= 256 and rng.random() < 0.5:
            table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
            if rng.random() < 0.7:
                shared = int(rng.integers(1, width + 1))
                table[:, :shared] = table[0, :shared]
            runs = cabi.prefix_runs(lib, table)
        hints = int(rng.integers(0, 4))
        merge = int(rng.integers(0, 2))
        args = (q_dtype, kv_dtype, batch, kv * group, kv, dim, page, width, batch * width, splits, split, merge, hints,
                bounds, 256, runs)
        try:
            plan = cabi.launch_plan(lib, *args)
        except ValueError:
            continue  # a shape the checks reject (for example the shared merge's state limit)
        planned += 1
        where = f"case {case}: {args[:13]} bounds kind {bounds_kind} runs {runs is not None} -> {plan}"
        c = plan["kernel_split_tokens"] // split
        assert plan["kernel_split_tokens"] == c * split and c >= 1 and c & (c - 1) == 0, where
        assert plan["kernel_splits"] == -(-splits // c) and plan["kernel_splits"] <= splits, where
        assert plan["launches"] in (1, 2), where
        assert 1 <= plan["grid_x"] < 1 << 32 and 1 <= plan["grid_y"] <= 65535 and 1 <= plan["grid_z"] <= 65535, where
        assert 1 <= plan["waves_per_workgroup"] <= 16, where
        assert 0 <= plan["shared_prefix_items"] <= 128, where
        if runs is None or bounds is None or q_dtype == cabi.PD_DTYPE_F32:
            assert plan["shared_prefix_items"] == 0, where
        if q_dtype == cabi.PD_DTYPE_F32 or bounds is None:
            assert c == 1, where
        grouped += plan["shared_prefix_items"] > 0
    assert planned > 2000 and grouped >= 5, (planned, grouped)
