"""GPU parity of the paged KV-cache append against the oracle's scatter.

The append moves bytes only, so the cache is compared bit for bit with
``oracle.fp64.scatter_tokens`` / ``append_advance`` on the same inputs; the
captured append + decode loop is checked against the FP64 attention oracle.
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle import fp64  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan, append_kv  # noqa: E402
from paged_decode.workload import make_tensors  # noqa: E402

pytestmark = pytest.mark.gpu


def cache_pair(layout, dtype, seed):
    _, k, v = make_tensors(layout, dtype=dtype, seed=seed)
    return k, v


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("dim,page_size", [(64, 16), (128, 32)])
@pytest.mark.parametrize("tokens", [1, 3])
def test_append_at_positions_matches_scatter(dtype, dim, page_size, tokens):
    announce(f"append positions dtype={dtype} dim={dim} page={page_size} tokens={tokens}")
    layout = Layout(5, 8, 2, dim, page_size, 24)
    k, v = cache_pair(layout, dtype, 31)
    rng = np.random.default_rng(tokens + dim)
    table = rng.permutation(24)[:20].reshape(5, 4).astype(np.int32)
    table[1, 2] = -1        # padding id: skipped
    table[3, 0] = 1 << 20   # id past the cache: skipped
    capacity = 4 * page_size
    positions = np.array([0, 2 * page_size - 1, capacity - 2, page_size - 1, -1], dtype=np.int32)
    k_new = torch.randn((5, tokens, 2, dim), device="cuda").to(dtype)
    v_new = torch.randn((5, tokens, 2, dim), device="cuda").to(dtype)
    expected_k = fp64.scatter_tokens(k.cpu().numpy(), table, positions, k_new.cpu().numpy())
    expected_v = fp64.scatter_tokens(v.cpu().numpy(), table, positions, v_new.cpu().numpy())
    append_kv(layout, k, v, torch.from_numpy(table).cuda(), torch.from_numpy(positions).cuda(), k_new, v_new)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(k.cpu().numpy(), expected_k)
    np.testing.assert_array_equal(v.cpu().numpy(), expected_v)


@pytest.mark.parametrize("tokens", [1, 2])
def test_advance_is_all_or_nothing_and_updates_lengths(tokens):
    announce(f"append advance tokens={tokens}")
    layout = Layout(4, 8, 2, 128, 16, 16)
    table = np.arange(16, dtype=np.int32).reshape(4, 4)
    table[2, 3] = -1                                         # seq 2 cannot grow into its 4th page
    lengths = np.array([5, 63, 47, 64], dtype=np.int32)      # seq 3 is full
    plan = DecodePlan(layout, table, lengths, max_context=64)
    k, v = cache_pair(layout, torch.float16, 5)
    k_new = torch.randn((4, tokens, 2, 128), device="cuda").half()
    v_new = torch.randn((4, tokens, 2, 128), device="cuda").half()
    expected_k, grown = fp64.append_advance(k.cpu().numpy(), table, lengths, k_new.cpu().numpy())
    expected_v, _ = fp64.append_advance(v.cpu().numpy(), table, lengths, v_new.cpu().numpy())
    plan.append(k, v, k_new if tokens > 1 else k_new[:, 0], v_new if tokens > 1 else v_new[:, 0])
    torch.cuda.synchronize()
    np.testing.assert_array_equal(k.cpu().numpy(), expected_k)
    np.testing.assert_array_equal(v.cpu().numpy(), expected_v)
    np.testing.assert_array_equal(plan._lengths.cpu().numpy(), grown)
    assert grown[0] == 5 + tokens and grown[2] == 47 + (tokens if tokens == 1 else 0) and grown[3] == 64


@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_captured_decode_loop_append_then_attend(merge):
    """One graph = append this step's K/V, then decode; replayed step after step."""
    announce(f"captured decode loop merge={merge}")
    layout = Layout(3, 16, 4, 128, 16, 3 * 16)
    table = np.arange(3 * 16, dtype=np.int32).reshape(3, 16)
    lengths = np.array([100, 1, 250], dtype=np.int32)
    plan = DecodePlan(layout, table, lengths, split_tokens=64, merge=merge, max_context=256)
    q, k, v = make_tensors(layout, seed=77)
    q_step = torch.empty_like(q)
    k_step = torch.empty((3, 4, 128), device="cuda", dtype=torch.float16)
    v_step = torch.empty_like(k_step)
    plan.run(q, k, v)  # warm up before capture (reads only)
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
    # Capture records work without running it: the cache and lengths are untouched.
    host_k, host_v = (t.cpu().numpy() for t in (k, v))
    host_lengths = lengths.copy()
    rng = np.random.default_rng(3)
    for step in range(6):
        qs = rng.standard_normal(q.shape).astype(np.float16)
        ks = rng.standard_normal(k_step.shape).astype(np.float16)
        vs = rng.standard_normal(v_step.shape).astype(np.float16)
        q_step.copy_(torch.from_numpy(qs))
        k_step.copy_(torch.from_numpy(ks))
        v_step.copy_(torch.from_numpy(vs))
        graph.replay()
        torch.cuda.synchronize()
        host_k, _ = fp64.append_advance(host_k, table, host_lengths, ks[:, None])
        host_v, host_lengths = fp64.append_advance(host_v, table, host_lengths, vs[:, None])
        expected = fp64.dense_attention(qs, host_k, host_v, table, host_lengths)
        assert_parity(out.cpu().numpy(), expected, torch.float16)
        np.testing.assert_array_equal(plan._lengths.cpu().numpy(), host_lengths)
    np.testing.assert_array_equal(k.cpu().numpy(), host_k)
    assert host_lengths.tolist() == [106, 7, 256]


@pytest.mark.parametrize("lengths0", [[0, 40, 0, 3000], [300, 290, 280, 310]], ids=["work-list", "rectangular-tails"])
def test_captured_growth_far_past_the_captured_bounds(lengths0):
    """A graph captured at short lengths keeps decoding correctly while its appends
    grow the sequences thousands of tokens past the bounds baked into the capture:
    the partitions past them run as tail items (at most four per sequence, here 16
    partitions each) in both grids that carry them, the work list (very ragged
    lengths) and the rectangular grid with tail slices."""
    announce(f"captured growth past the captured bounds, lengths {lengths0}")
    layout = Layout(4, 8, 2, 128, 16, 4 * 512)
    rng = np.random.default_rng(11)
    table = rng.permutation(4 * 512).reshape(4, 512).astype(np.int32)
    lengths = np.array(lengths0, dtype=np.int32)
    plan = DecodePlan(layout, table, lengths, split_tokens=128, max_context=8192)
    assert plan.splits == 64 and plan.launches(torch.float16) == 2
    q, k, v = make_tensors(layout, seed=78)
    tokens = 512
    q_step = torch.empty_like(q)
    k_step = torch.empty((4, tokens, 2, 128), device="cuda", dtype=torch.float16)
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
    for step in range(8):
        qs = rng.standard_normal(q.shape).astype(np.float16)
        ks = rng.standard_normal(k_step.shape).astype(np.float16)
        vs = rng.standard_normal(v_step.shape).astype(np.float16)
        q_step.copy_(torch.from_numpy(qs))
        k_step.copy_(torch.from_numpy(ks))
        v_step.copy_(torch.from_numpy(vs))
        graph.replay()
        torch.cuda.synchronize()
        host_k, _ = fp64.append_advance(host_k, table, host_lengths, ks, max_context=8192)
        host_v, host_lengths = fp64.append_advance(host_v, table, host_lengths, vs, max_context=8192)
        expected = fp64.dense_attention(qs, host_k, host_v, table, host_lengths)
        assert_parity(out.cpu().numpy(), expected, torch.float16)
        np.testing.assert_array_equal(plan._lengths.cpu().numpy(), host_lengths)
    assert (host_lengths == np.array(lengths0) + 8 * tokens).all()


@pytest.mark.parametrize("max_context", [None, 132])
def test_captured_appends_stop_at_the_reserved_context(max_context):
    """Appends never grow a sequence past the context the plan's partitions
    cover: with the default plan (reserved context = the longest initial
    length, 100) the length stays at 100; with 132 reserved it stops at 132.
    Every replay's output matches the FP64 oracle on the tokens that are live."""
    announce(f"captured appends bounded by the reserved context, max_context={max_context}")
    layout = Layout(1, 8, 2, 128, 16, 16)
    table = np.arange(16, dtype=np.int32)[None, ::-1].copy()    # 16 pages x 16 tokens: room for 256
    lengths = np.array([100], dtype=np.int32)
    plan = DecodePlan(layout, table, lengths, split_tokens=64, max_context=max_context)
    limit = plan.context_capacity
    assert limit == (100 if max_context is None else 132)
    q, k, v = make_tensors(layout, seed=91)
    k_step = torch.empty((1, 2, 128), device="cuda", dtype=torch.float16)
    v_step = torch.empty_like(k_step)
    plan.run(q, k, v)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            plan.append(k, v, k_step, v_step)
            out = plan.run(q, k, v)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    host_q = q.cpu().numpy()
    host_k, host_v = (t.cpu().numpy() for t in (k, v))
    host_lengths = lengths.copy()
    rng = np.random.default_rng(17)
    for step in range(40):
        ks = rng.standard_normal(k_step.shape).astype(np.float16)
        vs = rng.standard_normal(v_step.shape).astype(np.float16)
        k_step.copy_(torch.from_numpy(ks))
        v_step.copy_(torch.from_numpy(vs))
        graph.replay()
        torch.cuda.synchronize()
        host_k, _ = fp64.append_advance(host_k, table, host_lengths, ks[:, None], max_context=limit)
        host_v, host_lengths = fp64.append_advance(host_v, table, host_lengths, vs[:, None], max_context=limit)
        np.testing.assert_array_equal(plan._lengths.cpu().numpy(), host_lengths)
        expected = fp64.dense_attention(host_q, host_k, host_v, table, host_lengths)
        assert_parity(out.cpu().numpy(), expected, torch.float16)
    assert host_lengths.tolist() == [min(limit, 140)]
    np.testing.assert_array_equal(k.cpu().numpy(), host_k)
    np.testing.assert_array_equal(v.cpu().numpy(), host_v)
