"""Whole-row launches: calls whose rows hold at most 128 KB of K and V per
(sequence, KV head) run as one launch that folds each row's states in LDS and
writes the output, instead of a partition launch and a merge launch.

Checked against the FP64 oracle on exactly the values the device holds, for
every storage format, head layouts that leave part of a head tile empty, empty
and one-token rows, invalid page ids inside live ranges, the size bound on
both sides, and graph replay; the plan's workspace must stay untouched, and
the result must agree with the two-launch path (partition stage, then merge
stage) to FP32 rounding.
"""
import ctypes

import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode import cabi  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import host_tensors  # noqa: E402

pytestmark = pytest.mark.gpu

FORMATS = [
    (torch.float32, None),
    (torch.float16, None),
    (torch.bfloat16, None),
    (torch.float16, torch.float8_e4m3fn),
    (torch.bfloat16, torch.float8_e5m2),
]

# (batch, query heads, KV heads, head_dim, page, pages per row, lengths, split_tokens):
# at most 128 tokens per row, so that even FP32 K/V at head_dim 128 stays within 128 KB.
SHAPES = [
    (4, 8, 2, 64, 16, 8, [0, 1, 17, 128], 128),      # one partition per row, an empty row
    (3, 20, 4, 128, 32, 4, [128, 77, 5], 32),        # group of 5 in a tile of 8, four partitions
    (6, 16, 1, 64, 16, 8, [128, 0, 3, 100, 128, 64], 48),  # a full 16-head tile (MQA)
    (2, 35, 5, 64, 16, 4, [64, 33], 16),             # group of 7, partitions of one page
]


def device_inputs(layout, q_dtype, kv_dtype, seed):
    """Device tensors in the formats, per-tensor scales, and the exact float64 values."""
    q, k, v = host_tensors(layout, dtype=np.float32, seed=seed)
    qt = torch.from_numpy(q).to(q_dtype)
    if kv_dtype is None:
        kt, vt, k_scale, v_scale = torch.from_numpy(k).to(q_dtype), torch.from_numpy(v).to(q_dtype), 1.0, 1.0
    else:
        largest = float(torch.finfo(kv_dtype).max)
        k_scale, v_scale = float(np.abs(k).max()) / largest, float(np.abs(v).max()) / largest
        kt = (torch.from_numpy(k) / k_scale).to(kv_dtype)
        vt = (torch.from_numpy(v) / v_scale).to(kv_dtype)
    exact = (qt.double().numpy(), kt.double().numpy() * k_scale, vt.double().numpy() * v_scale)
    return (qt.cuda(), kt.cuda(), vt.cuda()), (k_scale, v_scale), exact


def bar(q_dtype):
    return torch.float32 if q_dtype == torch.float32 else torch.float16


def problem(shape, seed):
    batch, heads, kv_heads, dim, page, width, lengths, split = shape
    layout = Layout(batch, heads, kv_heads, dim, page, batch * width)
    table = np.random.default_rng(seed).permutation(batch * width).reshape(batch, width).astype(np.int32)
    return layout, table, np.array(lengths, dtype=np.int32), split


@pytest.mark.parametrize("q_dtype,kv_dtype", FORMATS)
@pytest.mark.parametrize("shape", SHAPES, ids=["s1-empty", "gqa5-d128-p32", "mqa16", "gqa7-page-parts"])
@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_whole_rows_match_oracle(q_dtype, kv_dtype, shape, merge):
    announce(f"whole rows q={q_dtype} kv={kv_dtype} shape={shape} merge={merge}")
    layout, table, lengths, split = problem(shape, seed=shape[3] + shape[1])
    (q, k, v), (k_scale, v_scale), exact = device_inputs(layout, q_dtype, kv_dtype, seed=shape[1])
    plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
    assert plan.launches(q.dtype, k.dtype) == 1
    plan._numerator.fill_(float("nan"))
    plan._stats.fill_(float("nan"))
    out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).clone()
    torch.cuda.synchronize()
    actual = out.cpu().numpy()
    assert_parity(actual, dense_attention(*exact, table, lengths), bar(q_dtype))
    for b in np.flatnonzero(lengths == 0):
        np.testing.assert_array_equal(actual[b], 0.0)
    # The whole-row launch writes no states.
    assert torch.isnan(plan._numerator).all() and torch.isnan(plan._stats).all()
    # The two-launch path on the same inputs: the same attention to FP32 rounding.
    plan.run_partial(q, k, v, k_scale=k_scale, v_scale=v_scale)
    staged = plan.run_merge().clone()
    torch.testing.assert_close(out, staged, rtol=2e-5, atol=2e-6)


def test_row_size_bound():
    """128 KB of K and V per row is one launch, one 16-token group more is two; both match the oracle."""
    for tokens, launches in ((512, 1), (528, 2)):
        announce(f"whole-row bound: {tokens} FP16 tokens at head_dim 64")
        layout = Layout(3, 8, 2, 64, 16, 3 * tokens // 16)
        table = np.arange(3 * tokens // 16, dtype=np.int32).reshape(3, tokens // 16)
        lengths = np.array([tokens, tokens - 100, 1], dtype=np.int32)
        (q, k, v), _, exact = device_inputs(layout, torch.float16, None, seed=tokens)
        plan = DecodePlan(layout, table, lengths, split_tokens=64)
        assert plan.launches(q.dtype) == launches
        assert_parity(plan.run(q, k, v).cpu().numpy(), dense_attention(*exact, table, lengths), torch.float16)


def test_whole_rows_skip_invalid_page_ids():
    """Page ids outside [0, physical_pages) inside live ranges are skipped, as in the two-launch path."""
    announce("whole rows: invalid page ids")
    lib = cabi.load()
    layout = Layout(2, 16, 4, 128, 16, 8)
    (q, k, v), (k_scale, v_scale), exact = device_inputs(layout, torch.bfloat16, torch.float8_e4m3fn, seed=71)
    table = np.array([[0, 1, 1 << 30, 2], [3, -7, 4, 5]], dtype=np.int32)
    lengths = np.array([64, 50], dtype=np.int32)
    splits, split_tokens = 2, 32
    args = (2, 16, 4, 128, 16, 4, 8, splits, split_tokens)
    assert cabi.launch_count(lib, cabi.PD_DTYPE_BF16, cabi.PD_DTYPE_FP8_E4M3, *args) == 1
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    numerator = torch.empty((2, 16, 4 * splits, 128), device="cuda")
    stats = torch.empty((2, 16, 4 * splits, 2), device="cuda")
    out = torch.full((2, 16, 128), float("nan"), device="cuda")
    status = lib.pd_decode_ex(q.data_ptr(), cabi.PD_DTYPE_BF16, k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_FP8_E4M3,
                              k_scale, v_scale, d_table.data_ptr(), d_lengths.data_ptr(), numerator.data_ptr(),
                              stats.data_ptr(), out.data_ptr(), *args, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_NONE,
                              None, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    # Equivalent valid problem: the tokens of the invalid pages removed.
    keep = [[0, 1, 3], [0, 2, 3]]
    qx, kx, vx = exact
    expected = np.zeros((2, 16, 128))
    for b in range(2):
        pos = [t for t in range(lengths[b]) if t // 16 in keep[b]]
        rows_k = np.stack([kx[table[b][t // 16], t % 16] for t in pos])
        rows_v = np.stack([vx[table[b][t // 16], t % 16] for t in pos])
        for h in range(16):
            s = rows_k[:, h // 4] @ qx[b, h] / np.sqrt(128)
            p = np.exp(s - s.max())
            expected[b, h] = p @ rows_v[:, h // 4] / p.sum()
    assert_parity(out.cpu().numpy(), expected, torch.float16)


@pytest.mark.parametrize("q_dtype", [torch.float32, torch.float16])
def test_whole_rows_graph_replay(q_dtype):
    """A captured whole-row call replays to the eager call's bits, with eager work between replays."""
    announce(f"whole rows graph replay {q_dtype}")
    layout, table, lengths, split = problem(SHAPES[1], seed=3)
    (q, k, v), _, _ = device_inputs(layout, q_dtype, None, seed=4)
    plan = DecodePlan(layout, table, lengths, split_tokens=split)
    assert plan.launches(q.dtype) == 1
    eager = plan.run(q, k, v).clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        plan.run(q, k, v)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            plan.run(q, k, v)
    torch.cuda.current_stream().wait_stream(side)
    for _ in range(3):
        plan._out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(plan._out, eager)
