"""Full decode calls over coarser partitions.

On grids with many waves per CU a full call (``DecodePlan.run``, ``pd_decode_ex``)
runs its partition and merge launches over partitions of c x split_tokens
tokens (``DecodePlan.kernel_split``), whose fewer states fit the plan's
workspace. Checked against the FP64 oracle on exactly the values the device
holds, for FP16, BF16 and FP8 K/V, both merges, GQA and MQA head tiles,
uniform and ragged lengths; against the stage entries over the same partitions
and over the plan's own split (both to FP32 rounding); with a
NaN-poisoned workspace; and under graph capture with appends that grow the
sequences far past the captured bounds, so that a replay runs the capture's
coarse partitions with tail items.
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle import fp64  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import host_tensors  # noqa: E402

pytestmark = pytest.mark.gpu

FORMATS = [
    (torch.float16, None),
    (torch.bfloat16, None),
    (torch.float16, torch.float8_e4m3fn),
]

# (batch, query heads, KV heads, head_dim, page, pages per row, lengths (None: ragged), split_tokens)
SHAPES = {
    "gqa4-uniform": (16, 32, 8, 128, 16, 128, 2048, 128),
    "gqa4-ragged-page32": (24, 32, 8, 128, 32, 128, None, 128),
    "mqa16-d64": (64, 16, 1, 64, 16, 128, 2048, 128),
}


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


def problem(name, seed):
    batch, heads, kv_heads, dim, page, width, length, split = SHAPES[name]
    rng = np.random.default_rng(seed)
    layout = Layout(batch, heads, kv_heads, dim, page, batch * width)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    if length is None:
        lengths = rng.integers(0, width * page + 1, size=batch).astype(np.int32)
        lengths[0], lengths[1] = width * page, 0
    else:
        lengths = np.full(batch, length, dtype=np.int32)
    return layout, table, lengths, split


@pytest.mark.parametrize("merge", ["serial", "shared"])
@pytest.mark.parametrize("q_dtype,kv_dtype", FORMATS)
@pytest.mark.parametrize("name", list(SHAPES))
def test_coarse_calls_match_oracle_and_stage_entries(name, q_dtype, kv_dtype, merge):
    announce(f"coarse split {name} q={q_dtype} kv={kv_dtype} merge={merge}")
    layout, table, lengths, split = problem(name, seed=len(name))
    (q, k, v), (k_scale, v_scale), exact = device_inputs(layout, q_dtype, kv_dtype, seed=layout.batch)
    plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
    kernel_splits, kernel_tokens = plan.kernel_split(q.dtype, k.dtype)
    announce(f"  plan split {plan.splits} x {split}, kernel split {kernel_splits} x {kernel_tokens}")
    assert kernel_tokens > split and kernel_tokens % split == 0 and kernel_splits * kernel_tokens >= plan.splits * split
    plan._numerator.fill_(float("nan"))
    plan._stats.fill_(float("nan"))
    out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).clone()
    torch.cuda.synchronize()
    actual = out.cpu().numpy()
    assert_parity(actual, fp64.dense_attention(*exact, table, lengths), torch.float16)
    for b in np.flatnonzero(lengths == 0):
        np.testing.assert_array_equal(actual[b], 0.0)
    # The states of the coarse partitions fill only the workspace's leading part.
    states = layout.batch * layout.query_heads * 4 * kernel_splits
    assert torch.isnan(plan._stats.view(-1)[states * 2:]).all()
    # The stage entries over the same partitions: the same partition launch; the
    # separate merge also reads the empty slots of combined quarters, so FP32 rounding.
    plan.run_partial(q, k, v, k_scale=k_scale, v_scale=v_scale)
    torch.testing.assert_close(plan.run_merge(), out, rtol=1e-5, atol=1e-6)
    # Over the plan's own, finer partitions: the same attention to FP32 rounding.
    ext, bounds = plan._extension, torch.from_numpy(lengths.copy())
    ext.partial(q, k, v, plan._table, plan._lengths, plan._numerator, plan._stats, split, k_scale, v_scale,
                plan._unshared_pages, plan._ragged_lengths, bounds)
    ext.merge(plan._numerator, plan._stats, plan._out, plan._lengths, layout.page_size, table.shape[1], split,
              int(plan.merge_implementation == "shared"))
    torch.testing.assert_close(plan._out, out, rtol=1e-4, atol=2e-5)


GROWTH = {
    # 16 sequences of 1024 tokens, split 128: a rectangular grid with tail slices.
    "uniform": (16, [1024] * 16, 128, 4096),
    # 8 long and 24 short sequences, split 64: very ragged, so a work list.
    "ragged-work-list": (32, [4000] * 8 + [100] * 24, 64, 8192),
}


@pytest.mark.parametrize("name", list(GROWTH))
def test_captured_coarse_call_with_growth_past_the_captured_bounds(name):
    """A graph captured while the bounds give a coarse split keeps decoding
    correctly while captured appends grow the sequences by 3072 tokens: the
    partitions past the captured bounds run as tail items of the coarse grid,
    a rectangular one with tail slices or a work list. Every replay is checked
    against the FP64 oracle."""
    batch, lengths0, split, max_context = GROWTH[name]
    announce(f"captured coarse call {name}, appends growing by 6 x 512 tokens")
    heads, kv_heads, dim, page, width = 32, 8, 128, 16, 512
    layout = Layout(batch, heads, kv_heads, dim, page, batch * width)
    rng = np.random.default_rng(17)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = np.array(lengths0, dtype=np.int32)
    plan = DecodePlan(layout, table, lengths, split_tokens=split, max_context=max_context)
    kernel_splits, kernel_tokens = plan.kernel_split(torch.float16)
    announce(f"  plan split {plan.splits} x {split}, kernel split at capture {kernel_splits} x {kernel_tokens}")
    assert kernel_tokens > split
    q, k, v = (torch.from_numpy(x).to(torch.float16).cuda() for x in host_tensors(layout, dtype=np.float32, seed=5))
    tokens = 512
    q_step = torch.empty_like(q)
    k_step = torch.empty((batch, tokens, kv_heads, dim), device="cuda", dtype=torch.float16)
    v_step = torch.empty_like(k_step)
    plan.run(q, k, v)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            plan.append(k, v, k_step, v_step)
            out = plan.run(q_step, k, v)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    host_k, host_v = (t.cpu().numpy() for t in (k, v))
    host_lengths = lengths.copy()
    for step in range(6):
        qs = rng.standard_normal(q.shape).astype(np.float16)
        ks = rng.standard_normal(k_step.shape).astype(np.float16)
        vs = rng.standard_normal(v_step.shape).astype(np.float16)
        q_step.copy_(torch.from_numpy(qs))
        k_step.copy_(torch.from_numpy(ks))
        v_step.copy_(torch.from_numpy(vs))
        graph.replay()
        torch.cuda.synchronize()
        host_k, _ = fp64.append_advance(host_k, table, host_lengths, ks, max_context=max_context)
        host_v, host_lengths = fp64.append_advance(host_v, table, host_lengths, vs, max_context=max_context)
        announce(f"  replay {step}: longest {int(host_lengths.max())}")
        assert_parity(out.cpu().numpy(), fp64.dense_attention(qs, host_k, host_v, table, host_lengths),
                      torch.float16)
        np.testing.assert_array_equal(plan._lengths.cpu().numpy(), host_lengths)
    assert (host_lengths == lengths + 6 * tokens).all()
