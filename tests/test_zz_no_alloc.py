"""pd_decode_scratch, the entry point that allocates nothing, through the C ABI.

Its partition states live in the library's static per-device scratch instead
of a caller workspace. Each case is checked against pd_decode_ex on a
NaN-filled caller workspace, bit for bit (same kernels, same launch shapes),
and against the FP64 oracle to the parity tolerances. Two calls run in a row,
the second on a smaller problem, so stale contents of the shared scratch from
the first call would show in the second.
"""
import ctypes

import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle import fp64  # noqa: E402
from paged_decode import cabi  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.workload import host_tensors  # noqa: E402

pytestmark = pytest.mark.gpu

CODES = {np.float16: cabi.PD_DTYPE_F16, np.float32: cabi.PD_DTYPE_F32}


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def problem(layout, dtype, lengths, seed):
    rng = np.random.default_rng(seed)
    width = layout.physical_pages // layout.batch
    table = rng.permutation(layout.physical_pages).reshape(layout.batch, width).astype(np.int32)
    q, k, v = host_tensors(layout, dtype=dtype, seed=seed)
    return table, np.asarray(lengths, dtype=np.int32), (q, k, v)


def dims(layout, width, splits, split_tokens, merge, hints):
    return (layout.batch, layout.query_heads, layout.kv_heads, layout.head_dim, layout.page_size, width,
            layout.physical_pages, splits, split_tokens, merge, hints)


def run_both(lib, layout, dtype, lengths, split_tokens, merge, hints, seed, with_bounds=False):
    """(scratch-entry output, workspace-entry output, FP64 oracle) for one problem;
    with_bounds passes the lengths as host length bounds to both entries."""
    table, lengths, host = problem(layout, dtype, lengths, seed)
    bounds = lengths.copy() if with_bounds else None
    bounds_ptr = None if bounds is None else bounds.ctypes.data
    q, k, v = (torch.from_numpy(x).cuda() for x in host)
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    splits = max(1, -(-int(lengths.max()) // split_tokens))
    code = CODES[dtype]
    args = dims(layout, table.shape[1], splits, split_tokens, merge, hints)
    out_scratch = torch.full((layout.batch, layout.query_heads, layout.head_dim), float("nan"), device="cuda")
    status = lib.pd_decode_scratch(q.data_ptr(), code, k.data_ptr(), v.data_ptr(), code, 1.0, 1.0,
                                   d_table.data_ptr(), d_lengths.data_ptr(), out_scratch.data_ptr(), *args,
                                   bounds_ptr, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    shape = (layout.batch, layout.query_heads, 4 * splits)
    num = torch.full((*shape, layout.head_dim), float("nan"), device="cuda")
    stats = torch.full((*shape, 2), float("nan"), device="cuda")
    out_ws = torch.full_like(out_scratch, float("nan"))
    status = lib.pd_decode_ex(q.data_ptr(), code, k.data_ptr(), v.data_ptr(), code, 1.0, 1.0, d_table.data_ptr(),
                              d_lengths.data_ptr(), num.data_ptr(), stats.data_ptr(), out_ws.data_ptr(), *args,
                              bounds_ptr, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    expected = fp64.dense_attention(*host, table, lengths)
    return out_scratch.cpu().numpy(), out_ws.cpu().numpy(), expected


def test_scratch_entry_matches_workspace_entry_twice_then_smaller():
    lib = cabi.load()
    # First call: Llama-3-8B head geometry, ragged lengths (one empty),
    # 4 x 32 rows of 4 x 16 states.
    announce("pd_decode_scratch call 1: B4 Hq32 Hkv8 D128 FP16, split 64, serial, unshared-pages hint")
    big = Layout(4, 32, 8, 128, 16, 4 * 64)
    a_scratch, a_ws, a_ref = run_both(lib, big, np.float16, [1024, 0, 517, 1000], 64, cabi.PD_MERGE_SERIAL,
                                      cabi.PD_HINT_UNSHARED_PAGES, seed=5)
    np.testing.assert_array_equal(a_scratch, a_ws)
    assert_parity(a_scratch, a_ref, np.float16)
    # Second call, smaller: FP32, fewer heads and states, shared merge. The
    # scratch still holds the first call's states; only its own are read.
    announce("pd_decode_scratch call 2: B2 Hq8 Hkv2 D64 FP32, split 32, shared merge")
    small = Layout(2, 8, 2, 64, 16, 2 * 16)
    b_scratch, b_ws, b_ref = run_both(lib, small, np.float32, [100, 256], 32, cabi.PD_MERGE_SHARED,
                                      cabi.PD_HINT_NONE, seed=0)
    np.testing.assert_array_equal(b_scratch, b_ws)
    assert_parity(b_scratch, b_ref, np.float32)


def test_scratch_entry_over_coarser_partitions_then_smaller():
    """With length bounds on a grid of many waves per CU, both entries run over
    coarser partitions than the caller's (pd_decode_kernel_split); the scratch
    entry still matches the workspace entry bit for bit, then a smaller call
    with bounds at the caller's split follows on the same scratch."""
    lib = cabi.load()
    big = Layout(16, 32, 8, 128, 16, 16 * 128)
    announce("pd_decode_scratch with bounds, call 1: B16 Hq32 Hkv8 D128 FP16 L2048, split 128, serial")
    kernel = cabi.kernel_split(lib, cabi.PD_DTYPE_F16, cabi.PD_DTYPE_F16, 16, 32, 8, 128, 16, 128, 16 * 128, 16, 128,
                               [2048] * 16)
    assert kernel[1] > 128, kernel
    a_scratch, a_ws, a_ref = run_both(lib, big, np.float16, [2048] * 16, 128, cabi.PD_MERGE_SERIAL,
                                      cabi.PD_HINT_UNSHARED_PAGES, seed=21, with_bounds=True)
    np.testing.assert_array_equal(a_scratch, a_ws)
    assert_parity(a_scratch, a_ref, np.float16)
    announce("pd_decode_scratch with bounds, call 2: B4 Hq32 Hkv8 D128 FP16 ragged, split 64, shared")
    small = Layout(4, 32, 8, 128, 16, 4 * 64)
    b_scratch, b_ws, b_ref = run_both(lib, small, np.float16, [1024, 0, 517, 1000], 64, cabi.PD_MERGE_SHARED,
                                      cabi.PD_HINT_NONE, seed=22, with_bounds=True)
    np.testing.assert_array_equal(b_scratch, b_ws)
    assert_parity(b_scratch, b_ref, np.float16)


def test_scratch_entry_rejects_workspaces_beyond_the_scratch():
    """A request whose states exceed PD_SCRATCH_BYTES returns PD_ERR_SCRATCH and launches nothing."""
    announce("pd_decode_scratch oversized request")
    lib = cabi.load()
    layout = Layout(8, 64, 8, 128, 16, 8 * 256)
    table, lengths, host = problem(layout, np.float16, [4096] * 8, seed=2)
    q, k, v = (torch.from_numpy(x).cuda() for x in host)
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    splits, split_tokens = 64, 64          # 8 * 64 * 256 states of 520 B: 68 MB > 32 MiB
    out = torch.full((8, 64, 128), float("nan"), device="cuda")
    status = lib.pd_decode_scratch(q.data_ptr(), cabi.PD_DTYPE_F16, k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F16,
                                   1.0, 1.0, d_table.data_ptr(), d_lengths.data_ptr(), out.data_ptr(),
                                   *dims(layout, 256, splits, split_tokens, cabi.PD_MERGE_SERIAL, 0), None, stream())
    assert status == cabi.PD_ERR_SCRATCH
    assert "scratch" in cabi.status_string(lib, status)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    # The same problem at split 256 (16 splits, 17 MB of states) fits and runs.
    status = lib.pd_decode_scratch(q.data_ptr(), cabi.PD_DTYPE_F16, k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F16,
                                   1.0, 1.0, d_table.data_ptr(), d_lengths.data_ptr(), out.data_ptr(),
                                   *dims(layout, 256, 16, 256, cabi.PD_MERGE_SERIAL, 0), None, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    assert_parity(out.cpu().numpy(), fp64.dense_attention(*host, table, lengths), np.float16)


def test_scratch_entry_allocates_nothing_and_replays_in_a_graph():
    """What the entry exists for: after one uncaptured call on a device (which
    looks up the scratch's address), a call changes no device allocation
    (hipMemGetInfo's free bytes are unchanged), and a call captured in a
    hipGraph on a side stream replays bit for bit like the eager call, with
    the program's own eager work between the replays."""
    lib = cabi.load()
    layout = Layout(8, 32, 8, 128, 16, 8 * 128)
    lengths = np.array([2048, 1999, 0, 2048, 1024, 77, 2048, 1500], dtype=np.int32)
    table, lengths, host = problem(layout, np.float16, lengths, seed=31)
    bounds = lengths.copy()
    q, k, v = (torch.from_numpy(x).cuda() for x in host)
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    args = dims(layout, table.shape[1], 16, 128, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_UNSHARED_PAGES)
    eager = torch.full((8, 32, 128), float("nan"), device="cuda")
    graph_out = torch.full_like(eager, float("nan"))

    def call(out):
        status = lib.pd_decode_scratch(q.data_ptr(), cabi.PD_DTYPE_F16, k.data_ptr(), v.data_ptr(),
                                       cabi.PD_DTYPE_F16, 1.0, 1.0, d_table.data_ptr(), d_lengths.data_ptr(),
                                       out.data_ptr(), *args, bounds.ctypes.data, stream())
        assert status == cabi.PD_OK, cabi.status_string(lib, status)

    announce("pd_decode_scratch: warm-up call, then a call between two hipMemGetInfo readings")
    call(eager)
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    call(eager)
    torch.cuda.synchronize()
    free_after, _ = torch.cuda.mem_get_info()
    assert free_after == free_before
    assert_parity(eager.cpu().numpy(), fp64.dense_attention(*host, table, lengths), np.float16)

    announce("pd_decode_scratch: captured in a hipGraph on a side stream, replayed 4 times")
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            call(graph_out)
    torch.cuda.synchronize()
    for replay in range(4):
        graph_out.fill_(float("nan"))
        scribble = torch.randn(1 << 20, device="cuda").sum()  # the program's own eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.isfinite(scribble)
        assert torch.equal(graph_out, eager), f"replay {replay}"
