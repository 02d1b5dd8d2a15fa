"""GPU parity of shared-prefix items against the FP64 oracle.

A work-list launch with prefix runs (``pd_prefix_runs``) and host bounds
scores each partition inside several sequences' common prefix once for up to
16 / GT of them (``plan_prefix_items``). Each case first checks, through the
launch plan, that the items are formed, then compares the output with
``oracle.fp64.dense_attention`` on the same inputs, and with the same call
made without runs (one read per sequence). The kernel's page check makes the
result independent of the runs: stale runs, a graph captured before a
``refresh`` that changes the sharing, and a captured append loop that grows
sequences from the shared prefix onto pages of their own stay exact.
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle import fp64  # noqa: E402
from paged_decode import cabi  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import host_tensors, make_tensors, make_workload  # noqa: E402

pytestmark = pytest.mark.gpu


def shared_table(rng, batch, width, classes):
    """Shuffled private pages, then for each (leader, members, pages) the members'
    first `pages` entries set to the leader's."""
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    for leader, members, pages in classes:
        for b in members:
            table[b, :pages] = table[leader, :pages]
    return table


def padded(table, lengths, page_size):
    table = table.copy()
    for b, length in enumerate(lengths):
        table[b, (int(length) + page_size - 1) // page_size:] = -1
    return table


def inputs(layout, q_dtype, kv_dtype, seed):
    """Device q, k, v in the formats, their scales, and the exact float64 values."""
    q, k, v = host_tensors(layout, dtype=np.float32, seed=seed)
    qt = torch.from_numpy(q).to(q_dtype)
    if kv_dtype is None:
        kt, vt, k_scale, v_scale = torch.from_numpy(k).to(q_dtype), torch.from_numpy(v).to(q_dtype), 1.0, 1.0
    else:
        largest = float(torch.finfo(kv_dtype).max)
        k_scale, v_scale = float(np.abs(k).max()) / largest, float(np.abs(v).max()) / largest
        kt, vt = (torch.from_numpy(k) / k_scale).to(kv_dtype), (torch.from_numpy(v) / v_scale).to(kv_dtype)
    exact = (qt.double().numpy(), kt.double().numpy() * k_scale, vt.double().numpy() * v_scale)
    return (qt.cuda(), kt.cuda(), vt.cuda()), (k_scale, v_scale), exact


def case(name):
    """(layout, table, lengths, split_tokens, q dtype, K/V dtype or None)."""
    rng = np.random.default_rng(sum(map(ord, name)))
    if name == "workload ragged+shared B16 GQA4 page 32":
        w = make_workload("ragged_shared_b16")
        return w.layout, w.table, w.lengths, w.split_tokens, torch.float16, None
    if name == "mha B24 D64 (16 members per item)":
        lengths = np.concatenate([[4096], rng.integers(520, 1520, 23)]).astype(np.int32)
        table = shared_table(rng, 24, 256, [(0, range(1, 24), 32)])
        return Layout(24, 8, 8, 64, 16, 24 * 256), padded(table, lengths, 16), lengths, 64, torch.float16, None
    if name == "gqa8 B6 bf16 (2 members per item)":
        lengths = np.array([2048, 400, 700, 300, 650, 520], dtype=np.int32)
        table = shared_table(rng, 6, 128, [(0, range(1, 6), 16)])
        return Layout(6, 16, 2, 128, 16, 6 * 128), padded(table, lengths, 16), lengths, 64, torch.bfloat16, None
    if name == "gqa4 B16 fp8 e4m3 K/V":
        lengths = np.concatenate([[8192], rng.integers(0, 3000, 15)]).astype(np.int32)
        table = shared_table(rng, 16, 256, [(0, range(1, 16), 64)])
        return Layout(16, 32, 8, 128, 32, 16 * 256), padded(table, lengths, 32), lengths, 128, torch.float16, \
            torch.float8_e4m3fn
    if name == "two classes B16 GQA4":
        lengths = (600 + 97 * np.arange(16)).astype(np.int32)
        lengths[0] = 8192
        table = shared_table(rng, 16, 256, [(0, range(1, 8), 48), (8, range(9, 16), 24), (8, [12], 40)])
        table[3, 10:48] = rng.permutation(np.arange(16 * 256, 17 * 256))[:38]  # diverges after 10 pages
        return Layout(16, 32, 8, 128, 32, 17 * 256), padded(table, lengths, 32), lengths, 128, torch.float16, None
    if name == "samples B32 L4096 50% shared (equal lengths)":
        lengths = np.full(32, 4096, dtype=np.int32)
        table = shared_table(rng, 32, 256, [(0, range(1, 32), 128)])
        return Layout(32, 32, 8, 128, 16, 32 * 256), table, lengths, 256, torch.float16, None
    if name == "samples B16 L4096 50% shared (half the coarse split)":
        lengths = np.full(16, 4096, dtype=np.int32)
        table = shared_table(rng, 16, 256, [(0, range(1, 16), 128)])
        return Layout(16, 32, 8, 128, 16, 16 * 256), table, lengths, 256, torch.float16, None
    if name == "samples B8 L8192 50% shared bf16 (half the coarse split)":
        lengths = np.full(8, 8192, dtype=np.int32)
        table = shared_table(rng, 8, 512, [(0, range(1, 8), 256)])
        return Layout(8, 32, 8, 128, 16, 8 * 512), table, lengths, 256, torch.bfloat16, None
    if name == "samples B16 L4096 50% shared fp8 e4m3 K/V":
        lengths = np.full(16, 4096, dtype=np.int32)
        table = shared_table(rng, 16, 256, [(0, range(1, 16), 128)])
        return Layout(16, 32, 8, 128, 16, 16 * 256), table, lengths, 256, torch.float16, torch.float8_e4m3fn
    raise KeyError(name)


# Cases whose full call runs over half the partition span it takes without
# runs (prefix_finer_split): 512 tokens instead of 1024.
FINER = {"samples B16 L4096 50% shared (half the coarse split)": 512, "samples B16 L4096 50% shared fp8 e4m3 K/V": 512,
         "samples B8 L8192 50% shared bf16 (half the coarse split)": 512}


CASES = ["workload ragged+shared B16 GQA4 page 32", "mha B24 D64 (16 members per item)",
         "gqa8 B6 bf16 (2 members per item)", "gqa4 B16 fp8 e4m3 K/V", "two classes B16 GQA4",
         "samples B32 L4096 50% shared (equal lengths)", "samples B16 L4096 50% shared (half the coarse split)",
         "samples B8 L8192 50% shared bf16 (half the coarse split)", "samples B16 L4096 50% shared fp8 e4m3 K/V"]


@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_shared_prefix_items_match_the_oracle(name, merge):
    layout, table, lengths, split, q_dtype, kv_dtype = case(name)
    (q, k, v), (k_scale, v_scale), exact = inputs(layout, q_dtype, kv_dtype, seed=len(name))
    plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
    launch = plan.launch_plan(q.dtype, k.dtype)
    announce(f"shared prefix {name} merge={merge}: {launch['shared_prefix_items']} items, "
             f"kernel split {launch['kernel_split']}")
    assert launch["shared_prefix_items"] > 0 and launch["grid_kind"] == "work list"
    if name in FINER:
        assert launch["kernel_split"][1] == FINER[name] and plan.kernel_split(q.dtype)[1] == FINER[name]
    out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).clone()
    expected = fp64.dense_attention(*exact, table, lengths)
    assert_parity(out.cpu().numpy(), expected, torch.float16)
    # The same call reading every sequence's pages itself (no runs).
    ext = plan._extension
    alone = torch.empty_like(out)
    ext.decode(q, k, v, plan._table, plan._lengths, plan._numerator, plan._stats, alone, split, plan._merge_mode,
               k_scale, v_scale, plan._unshared_pages, plan._ragged_lengths, plan._length_bounds(), None)
    torch.testing.assert_close(out, alone, rtol=0, atol=2e-5)
    # The staged entries over the same partitions agree too.
    plan.run_partial(q, k, v, k_scale=k_scale, v_scale=v_scale)
    torch.testing.assert_close(plan.run_merge().clone(), out, rtol=0, atol=2e-5)


def test_stale_runs_stay_correct():
    """Runs that claim every row equal to its leader's over the whole table:
    items then reach pages the members do not map, the page check sends those
    members to passes over their own rows, and the output is still exact."""
    layout, table, lengths, split, q_dtype, kv_dtype = case("two classes B16 GQA4")
    (q, k, v), (k_scale, v_scale), exact = inputs(layout, q_dtype, kv_dtype, seed=3)
    plan = DecodePlan(layout, table, lengths, split_tokens=split)
    lib = cabi.load()
    stale = cabi.prefix_runs(lib, table).reshape(-1, 2)
    stale[stale[:, 0] >= 0, 1] = table.shape[1]
    stale = torch.from_numpy(stale.reshape(-1).copy())
    announce("shared prefix: stale runs")
    out = torch.empty((layout.batch, layout.query_heads, layout.head_dim), device="cuda")
    plan._extension.decode(q, k, v, plan._table, plan._lengths, plan._numerator, plan._stats, out, split,
                           plan._merge_mode, k_scale, v_scale, False, plan._ragged_lengths, plan._length_bounds(),
                           stale)
    assert_parity(out.cpu().numpy(), fp64.dense_attention(*exact, table, lengths), torch.float16)


def test_graph_captured_before_a_refresh_that_changes_the_sharing():
    """A graph captured with shared-prefix items keeps them after ``refresh``
    (the launch arguments are the capture's). Refreshing to a table with no
    shared pages, then to one with a shorter shared prefix and new lengths,
    must still give the oracle's output on every replay."""
    layout, table, lengths, split, q_dtype, _ = case("mha B24 D64 (16 members per item)")
    q, k, v = make_tensors(layout, seed=23)
    host_q, host_k, host_v = (t.cpu().numpy() for t in (q, k, v))
    plan = DecodePlan(layout, table, lengths, split_tokens=split, max_context=4096)
    assert plan.launch_plan(q.dtype)["shared_prefix_items"] > 0
    plan.run(q, k, v)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = plan.run(q, k, v)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    rng = np.random.default_rng(29)
    private = padded(rng.permutation(layout.physical_pages)[:24 * 256].reshape(24, 256).astype(np.int32), lengths,
                     16)
    shorter_lengths = np.concatenate([[4096], rng.integers(0, 1500, 23)]).astype(np.int32)
    shorter = padded(shared_table(rng, 24, 256, [(0, range(1, 24), 7)]), shorter_lengths, 16)
    for step, (t, lens) in enumerate([(table, lengths), (private, lengths), (shorter, shorter_lengths),
                                      (table, lengths)]):
        plan.refresh(t, lens)
        for _ in range(2):
            graph.replay()
            torch.cuda.synchronize()
            announce(f"shared prefix: replay after refresh {step}")
            assert_parity(out.cpu().numpy(), fp64.dense_attention(host_q, host_k, host_v, t, lens), torch.float16)
        eager = plan.run(q, k, v).clone()  # eager work between replays
        torch.cuda.synchronize()
        assert_parity(eager.cpu().numpy(), fp64.dense_attention(host_q, host_k, host_v, t, lens), torch.float16)


def test_captured_append_loop_grows_members_past_the_shared_prompt():
    """Sequences start at the end of a shared 10-page prompt (160 tokens, which
    ends inside a 64-token partition), then a captured append + decode loop
    grows them onto pages of their own past the bounds baked into the capture.
    The partition holding the prompt's end stays a shared-prefix item; its page
    check sends each member's own tokens there to a pass over its own row."""
    announce("shared prefix: captured append loop past the shared prompt")
    layout = Layout(16, 8, 2, 128, 16, 16 * 64)
    rng = np.random.default_rng(37)
    table = shared_table(rng, 16, 64, [(0, range(1, 16), 10)])
    lengths = np.full(16, 160, dtype=np.int32)
    lengths[0] = 1024
    plan = DecodePlan(layout, table, lengths, split_tokens=64, max_context=1024)
    q, k, v = make_tensors(layout, seed=41)
    assert plan.launch_plan(q.dtype)["shared_prefix_items"] > 0
    k_step = torch.empty((16, 5, 2, 128), device="cuda", dtype=torch.float16)
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
    for step in range(12):
        ks = rng.standard_normal(k_step.shape).astype(np.float16)
        vs = rng.standard_normal(v_step.shape).astype(np.float16)
        ks[0], vs[0] = 0, 0  # sequence 0 (the prompt's owner) is full
        k_step.copy_(torch.from_numpy(ks))
        v_step.copy_(torch.from_numpy(vs))
        graph.replay()
        torch.cuda.synchronize()
        host_k, _ = fp64.append_advance(host_k, table, host_lengths, ks, max_context=1024)
        host_v, host_lengths = fp64.append_advance(host_v, table, host_lengths, vs, max_context=1024)
        np.testing.assert_array_equal(plan._lengths.cpu().numpy(), host_lengths)
        expected = fp64.dense_attention(host_q, host_k, host_v, table, host_lengths)
        assert_parity(out.cpu().numpy(), expected, torch.float16)
    assert (host_lengths[1:] == 160 + 12 * 5).all() and host_lengths[0] == 1024


def test_graph_captured_at_half_the_coarse_split_survives_refreshes():
    """Equal-length samples of a 50% shared prompt run over half the coarse
    split with shared-prefix items (512-token partitions instead of 1024). A
    graph captured so keeps that split and its items after ``refresh``: to a
    table with no shared pages, to ragged lengths under a shorter shared
    prompt, and back. Every replay, with eager calls in between (whose own
    plans follow each refresh), matches the FP64 oracle."""
    layout, table, lengths, split, _, _ = case("samples B16 L4096 50% shared (half the coarse split)")
    q, k, v = make_tensors(layout, seed=43)
    host_q, host_k, host_v = (t.cpu().numpy() for t in (q, k, v))
    plan = DecodePlan(layout, table, lengths, split_tokens=split)
    launch = plan.launch_plan(q.dtype)
    assert launch["kernel_split"][1] == 512 and launch["shared_prefix_items"] > 0
    announce("shared prefix: graph at half the coarse split, refreshed")
    plan.run(q, k, v)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            out = plan.run(q, k, v)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    rng = np.random.default_rng(47)
    private = rng.permutation(layout.physical_pages)[:16 * 256].reshape(16, 256).astype(np.int32)
    ragged = np.concatenate([[4096], rng.integers(0, 4097, 15)]).astype(np.int32)
    shorter = shared_table(rng, 16, 256, [(3, [b for b in range(16) if b != 3], 40)])
    for step, (t, lens) in enumerate([(table, lengths), (private, lengths), (shorter, ragged), (table, lengths)]):
        plan.refresh(t, lens)
        for _ in range(2):
            graph.replay()
            torch.cuda.synchronize()
            announce(f"shared prefix: replay at half the coarse split after refresh {step}")
            assert_parity(out.cpu().numpy(), fp64.dense_attention(host_q, host_k, host_v, t, lens), torch.float16)
        eager = plan.run(q, k, v).clone()
        torch.cuda.synchronize()
        assert_parity(eager.cpu().numpy(), fp64.dense_attention(host_q, host_k, host_v, t, lens), torch.float16)


PREFIX_STRESS_CASES = 240


def test_randomized_shared_prefixes():
    """Randomized sharing patterns against the FP64 oracle and the same call
    without runs: batches of 2 to 24, 1 to 8 KV heads with GQA groups 1 to 8
    (items form) or 16 (they do not), head dims 64 / 128, pages 16 / 32,
    splits 16 to 256, uniform, ragged or skewed lengths up to 1536 tokens,
    FP16 / BF16 / FP8-e4m3 K/V, one to three sharing classes with random
    leaders, members and shared page counts (some members diverging earlier),
    rows padded past their lengths or not, alternating merges."""
    rng = np.random.default_rng(13579)
    worst, grouped = 0.0, 0
    for seed in range(PREFIX_STRESS_CASES):
        batch = int(rng.choice([2, 3, 5, 8, 12, 16, 24]))
        kv = int(rng.choice([1, 2, 4, 8]))
        group = int(rng.choice([1, 2, 3, 4, 8, 16]))
        dim = int(rng.choice([64, 128]))
        page = int(rng.choice([16, 32]))
        split = int(rng.choice([16, 32, 64, 128, 256]))
        longest = int(rng.integers(64, 1537))
        width = -(-longest // page)
        kind = int(rng.choice(3, p=[0.2, 0.4, 0.4]))  # uniform, ragged, skewed
        lengths = np.full(batch, longest, dtype=np.int32)
        if kind == 1:
            lengths[1:] = rng.integers(0, longest + 1, batch - 1)
        elif kind == 2:
            lengths[1:] = rng.integers(0, longest // 2 + 1, batch - 1)
        classes = []
        for _ in range(int(rng.integers(1, 4))):
            leader = int(rng.integers(0, batch))
            pages = int(rng.integers(1, width + 1) if rng.random() < 0.3 else rng.integers(width // 4 + 1, width + 1))
            members = [b for b in range(batch) if b != leader and rng.random() < 2 / 3]
            classes.append((leader, members, pages))
        table = shared_table(rng, batch, width, [(leader, members, pages) for leader, members, pages in classes])
        for leader, members, pages in classes:  # a quarter of the members diverge earlier
            for b in members:
                if rng.random() < 0.25:
                    cut = int(rng.integers(0, pages + 1))
                    table[b, cut:pages] = rng.permutation(np.arange(batch * width, batch * width + width))[
                        :pages - cut]
        if rng.random() < 0.5:
            table = padded(table, lengths, page)
        layout = Layout(batch, kv * group, kv, dim, page, batch * width + width)
        fmt = str(rng.choice(["f16", "f16", "bf16", "e4m3"]))
        q_dtype = torch.bfloat16 if fmt == "bf16" else torch.float16
        kv_dtype = torch.float8_e4m3fn if fmt == "e4m3" else None
        (q, k, v), (k_scale, v_scale), exact = inputs(layout, q_dtype, kv_dtype, seed=seed + 30000)
        merge = ("serial", "shared")[seed % 2]
        plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
        items = plan.launch_plan(q.dtype, k.dtype)["shared_prefix_items"]
        grouped += items > 0
        if seed % 20 == 0:
            announce(f"shared prefix stress case {seed}: {grouped} with items so far, worst {worst:.3e}")
        out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).clone()
        expected = fp64.dense_attention(*exact, table, lengths)
        worst = max(worst, float(np.max(np.abs(out.cpu().numpy() - expected))))
        ext = plan._extension
        alone = torch.empty_like(out)
        ext.decode(q, k, v, plan._table, plan._lengths, plan._numerator, plan._stats, alone, split,
                   plan._merge_mode, k_scale, v_scale, plan._unshared_pages, plan._ragged_lengths,
                   plan._length_bounds(), None)
        try:
            assert_parity(out.cpu().numpy(), expected, torch.float16)
            torch.testing.assert_close(out, alone, rtol=0, atol=2e-5)
        except AssertionError as exc:
            raise AssertionError(f"case {seed}: {layout} split={split} {fmt} merge={merge} items={items} "
                                 f"lengths={lengths.tolist()} classes={[(l, len(m), p) for l, m, p in classes]}"
                                 ) from exc
    announce(f"shared prefix stress: {PREFIX_STRESS_CASES} cases, {grouped} with items, max abs error {worst:.3e}")
    assert grouped >= PREFIX_STRESS_CASES // 4
