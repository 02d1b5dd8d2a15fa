"""GPU parity of DecodePlan against the FP64 oracle.

Mirrors every case of reference tests/test_cuda.py (83 cases) with the stricter
tolerances of tests/gpu_util.py, and adds golden fixtures, non-finite-input
guards and the raw C-ABI path.
"""
import ctypes

import numpy as np
import pytest

from gpu_util import announce, assert_parity, host, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode import cabi  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import make_tensors, make_workload  # noqa: E402

pytestmark = pytest.mark.gpu


def oracle(q, k, v, table, lengths):
    return dense_attention(*host(q, k, v), table, lengths)


@pytest.mark.parametrize("merge", ["serial", "shared"])
@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("page_size", [16, 32])
@pytest.mark.parametrize("split", [1, 33, 256])
def test_ragged_decode(dim, dtype, page_size, split, merge):
    announce(f"ragged dim={dim} dtype={dtype} page={page_size} split={split} merge={merge}")
    layout = Layout(4, 8, 2, dim, page_size, 32)
    table = np.random.default_rng(5).permutation(32).reshape(4, 8).astype(np.int32)
    lengths = np.array([0, 1, page_size + 1, 127], dtype=np.int32)
    for b, length in enumerate(lengths):
        table[b, (int(length) + page_size - 1) // page_size:] = -1
    q, k, v = make_tensors(layout, dtype=dtype)
    plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
    actual = plan.run(q, k, v).cpu().numpy()
    assert_parity(actual, oracle(q, k, v, table, lengths), dtype)
    np.testing.assert_array_equal(actual[0], 0.0)


@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_nondefault_stream_and_graph_capture(merge):
    announce(f"graph capture merge={merge}")
    layout = Layout(1, 8, 2, 64, 16, 8)
    table, lengths = np.arange(8, dtype=np.int32)[None], np.array([127], dtype=np.int32)
    q, k, v = make_tensors(layout)
    plan = DecodePlan(layout, table, lengths, merge=merge)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        expected = plan.run(q, k, v).clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            output = plan.run(q, k, v)
        for _ in range(3):
            output.zero_()
            graph.replay()
            torch.testing.assert_close(output, expected, rtol=0, atol=0)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    assert_parity(expected.cpu().numpy(), oracle(q, k, v, table, lengths), torch.float16)


@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_large_logits_and_repeated_pages(merge):
    announce(f"large logits merge={merge}")
    layout = Layout(2, 8, 1, 128, 16, 4)
    table = np.array([[2, 0, 1, 3], [2, 0, 1, 3]], dtype=np.int32)
    lengths = np.array([64, 37], dtype=np.int32)
    q, k, v = make_tensors(layout, dtype=torch.float32)
    q *= 100
    plan = DecodePlan(layout, table, lengths, split_tokens=17, merge=merge)
    actual = plan.run(q, k, v).cpu().numpy()
    # Reference tolerance for this case (tests/test_cuda.py:64): scores reach
    # ~1e3, so FP32 rounding of the logits alone moves weights by ~1e-4.
    np.testing.assert_allclose(actual, oracle(q, k, v, table, lengths), atol=3e-3, rtol=3e-3)


def test_rejects_invalid_inputs():
    layout = Layout(1, 8, 2, 64, 16, 8)
    plan = DecodePlan(layout, np.arange(8, dtype=np.int32)[None], np.array([127]))
    q, k, v = make_tensors(layout)
    with pytest.raises(TypeError):
        plan.run(q.double(), k, v)
    with pytest.raises(ValueError):
        plan.run(q.transpose(1, 2), k, v)
    with pytest.raises(ValueError):
        plan.run(q.requires_grad_(), k, v)


@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_all_empty_contexts_and_long_partition_tail(merge):
    for lengths in (np.array([0, 0], dtype=np.int32), np.array([8193, 17], dtype=np.int32)):
        announce(f"empty/tail lengths={lengths.tolist()} merge={merge}")
        layout = Layout(2, 4, 4, 64, 16, 1026)
        table = np.arange(1026, dtype=np.int32).reshape(2, 513)
        q, k, v = make_tensors(layout, dtype=torch.float32)
        plan = DecodePlan(layout, table, lengths, split_tokens=257, merge=merge)
        actual = plan.run(q, k, v).cpu().numpy()
        assert_parity(actual, oracle(q, k, v, table, lengths), torch.float32)
        if not lengths.any():
            np.testing.assert_array_equal(actual, 0.0)


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_randomized_layout_and_content(seed, merge):
    rng = np.random.default_rng(seed)
    dim, page = int(rng.choice([64, 128])), int(rng.choice([16, 32]))
    heads = int(rng.choice([1, 4, 8]))
    kv_heads = int(rng.choice([h for h in [1, 2, 4, 8] if heads % h == 0]))
    layout = Layout(3, heads, kv_heads, dim, page, 20)
    lengths = np.array([0, int(rng.integers(1, 64)), 257], dtype=np.int32)
    table = rng.integers(0, 20, size=(3, (257 + page - 1) // page), dtype=np.int32)  # repeats allowed
    dtype = torch.float16 if seed % 2 else torch.float32
    q, k, v = make_tensors(layout, dtype=dtype, seed=seed + 200)
    if seed % 3 == 0:
        q.zero_()  # uniform attention: the mean of V over logical tokens
    split = int(rng.choice([1, 31, 128, 511]))
    announce(f"randomized seed={seed} merge={merge} {layout} split={split}")
    plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
    actual = plan.run(q, k, v).cpu().numpy()
    expected = oracle(q, k, v, table, lengths)
    assert_parity(actual, expected, dtype)
    if seed % 3 == 0:
        _, _, vh = host(q, k, v)
        for b in (1, 2):
            pos = np.arange(lengths[b])
            rows = vh[table[b][pos // page], pos % page].astype(np.float64)  # [len, Hkv, D]
            mean = rows.mean(axis=0)
            for h in range(heads):
                assert_parity(actual[b, h], mean[h // (heads // kv_heads)], dtype)


@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_changing_decode_across_page_boundaries(merge):
    layout = Layout(1, 4, 2, 64, 16, 4)
    table = np.array([[2, 0, 3, 1]], dtype=np.int32)
    q, k, v = make_tensors(layout, dtype=torch.float32, seed=333)
    for length in [0, 1, 15, 16, 17, 31, 32, 33, 63, 64]:
        announce(f"page boundary length={length} merge={merge}")
        q.add_(0.01)
        if length:
            page = int(table[0, (length - 1) // 16])
            v[page, (length - 1) % 16].mul_(0.9)
        plan = DecodePlan(layout, table, np.array([length]), split_tokens=13, merge=merge)
        actual = plan.run(q, k, v).cpu().numpy()
        assert_parity(actual, oracle(q, k, v, table, [length]), torch.float32)


def test_shared_merge_resource_bound_uses_explicit_fallback():
    layout = Layout(1, 4, 1, 64, 16, 70)
    table = np.arange(70, dtype=np.int32)[None]
    lengths = np.array([1100], dtype=np.int32)
    q, k, v = make_tensors(layout, dtype=torch.float32)
    plan = DecodePlan(layout, table, lengths, split_tokens=1, merge="shared")
    assert plan.merge_implementation == "serial_fallback"
    announce("shared-merge fallback split=1 len=1100")
    assert_parity(plan.run(q, k, v).cpu().numpy(), oracle(q, k, v, table, lengths), torch.float32)


@pytest.mark.parametrize("merge", ["serial", "shared"])
@pytest.mark.parametrize("dim", [64, 128])
def test_rows_of_thousands_of_states(dim, merge):
    """Split 1 at ~1000 tokens: 4000 states per row, merged over several load rounds."""
    announce(f"long rows dim={dim} merge={merge}")
    layout = Layout(4, 4, 2, dim, 16, 4 * 63)
    table = np.random.default_rng(9).permutation(4 * 63).reshape(4, 63).astype(np.int32)
    lengths = np.array([1000, 3, 0, 777], dtype=np.int32)
    q, k, v = make_tensors(layout, dtype=torch.float32)
    plan = DecodePlan(layout, table, lengths, split_tokens=1, merge=merge)
    assert plan.merge_implementation == merge
    actual = plan.run(q, k, v).cpu().numpy()
    assert_parity(actual, oracle(q, k, v, table, lengths), torch.float32)
    np.testing.assert_array_equal(actual[2], 0.0)


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_many_long_rows_and_reserved_context(dim, merge):
    """256 rows of up to 512 live states (split 16), in a plan sized for the
    longest sequence and in one reserving twice that: rows of more than 256
    states merged in several load rounds across a grid larger than the
    device's CUs. Both plans match the oracle and each other to FP32
    rounding: the reserved partitions are never written or read, but the
    call runs over coarser partitions (kernel_split) and the merge kernel's
    variant follows the allocated states per row, which differ."""
    announce(f"many long rows dim={dim} merge={merge}")
    layout = Layout(16, 16, 4, dim, 16, 16 * 256)
    rng = np.random.default_rng(31)
    table = rng.permutation(16 * 256).reshape(16, 256).astype(np.int32)
    lengths = rng.integers(0, 2049, size=16).astype(np.int32)
    lengths[0], lengths[1] = 2048, 0
    for b, n in enumerate(lengths):
        table[b, (n + 15) // 16:] = -1
    q, k, v = make_tensors(layout, dtype=torch.float16, seed=8)
    fitted = DecodePlan(layout, table, lengths, split_tokens=16, merge=merge)
    reserved = DecodePlan(layout, table, lengths, split_tokens=16, merge=merge, max_context=4096)
    assert fitted.splits == 128 and reserved.splits == 256
    out = fitted.run(q, k, v).clone()
    assert_parity(out.cpu().numpy(), oracle(q, k, v, table, lengths), torch.float16)
    torch.testing.assert_close(reserved.run(q, k, v), out, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(out[1].cpu().numpy(), 0.0)


@pytest.mark.parametrize("batch,query_heads,kv_heads", [(4, 32, 8), (8, 32, 4), (16, 16, 2)])
@pytest.mark.parametrize("shared_prefix", [False, True])
def test_mid_size_grids(batch, query_heads, kv_heads, shared_prefix):
    """Grids of one to two 8-wave workgroups per CU (4K context at split 256:
    256 of them for these head counts) run in workgroups of 2 KV heads x 2
    quarters with the quarters combined.
    Ragged lengths with a full and an empty row, prefix pages shared or not,
    both merges, against the oracle; the page-sharing hint (which switches
    the streamed loads) changes no bits."""
    announce(f"mid-size grid B{batch} Hq{query_heads}/Hkv{kv_heads} shared={shared_prefix}")
    width, page = 256, 16
    layout = Layout(batch, query_heads, kv_heads, 128, page, batch * width)
    rng = np.random.default_rng(batch + kv_heads)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = rng.integers(1, width * page + 1, size=batch).astype(np.int32)
    lengths[0], lengths[-1] = width * page, 0
    if shared_prefix:
        table[1:, :64] = table[0, :64]                             # every row's first 1024 tokens are row 0's
    for b, n in enumerate(lengths):
        table[b, (n + page - 1) // page:] = -1
    q, k, v = make_tensors(layout, dtype=torch.float16, seed=batch)
    expected = oracle(q, k, v, table, lengths)
    for merge in ("serial", "shared"):
        plan = DecodePlan(layout, table, lengths, split_tokens=256, merge=merge)
        assert plan.splits == 16 and plan._unshared_pages == (not shared_prefix)
        out = plan.run(q, k, v).clone()
        assert_parity(out.cpu().numpy(), expected, torch.float16)
        np.testing.assert_array_equal(out[-1].cpu().numpy(), 0.0)
        plan._unshared_pages = shared_prefix                       # the other streaming mode
        torch.testing.assert_close(plan.run(q, k, v), out, rtol=0, atol=0)


@pytest.mark.parametrize("batch,query_heads,kv_heads", [(16, 32, 8), (64, 16, 2)])
def test_ragged_lengths_hint(batch, query_heads, kv_heads):
    """Ragged batches of four 8-wave workgroups per CU (1024 at split 256):
    the plan sets the ragged-lengths hint and runs them in 2-head x 2-quarter
    workgroups; with the hint off they keep 8 waves. Both match the oracle
    and agree with each other to FP32 rounding."""
    announce(f"ragged-lengths hint B{batch} Hq{query_heads}/Hkv{kv_heads}")
    width, page = 256, 16
    layout = Layout(batch, query_heads, kv_heads, 128, page, batch * width)
    rng = np.random.default_rng(40 + kv_heads)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = rng.integers(0, width * page + 1, size=batch).astype(np.int32)
    lengths[0] = width * page
    for b, n in enumerate(lengths):
        table[b, (n + page - 1) // page:] = -1
    q, k, v = make_tensors(layout, dtype=torch.float16, seed=kv_heads)
    expected = oracle(q, k, v, table, lengths)
    plan = DecodePlan(layout, table, lengths, split_tokens=256)
    assert plan._ragged_lengths
    hinted = plan.run(q, k, v).clone()
    assert_parity(hinted.cpu().numpy(), expected, torch.float16)
    plan._ragged_lengths = False
    plain = plan.run(q, k, v)
    assert_parity(plain.cpu().numpy(), expected, torch.float16)
    torch.testing.assert_close(hinted, plain, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("batch,q_dtype,kv_dtype", [
    (32, torch.float16, None),                  # 2048 eight-wave workgroups: eight per CU, the rule's top
    (16, torch.bfloat16, None),
    (16, torch.float16, torch.float8_e4m3fn),
    (16, torch.bfloat16, torch.float8_e5m2),
])
def test_ragged_lengths_hint_formats(batch, q_dtype, kv_dtype):
    """The ragged-lengths hint at the top of its range (eight 8-wave workgroups per
    CU) and with BF16 and FP8 K/V: hinted (2-head x 2-quarter workgroups) and plain
    (8-wave) launches both match the FP64 oracle on the device's exact values and
    agree with each other to FP32 rounding."""
    from test_gpu_formats import quantized

    announce(f"ragged-lengths hint B{batch} q={q_dtype} kv={kv_dtype}")
    width, page = 256, 16
    layout = Layout(batch, 32, 8, 128, page, batch * width)
    rng = np.random.default_rng(60 + batch)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = rng.integers(0, width * page + 1, size=batch).astype(np.int32)
    lengths[0] = width * page
    for b, n in enumerate(lengths):
        table[b, (n + page - 1) // page:] = -1
    (q, k, v), (k_scale, v_scale), exact = quantized(layout, q_dtype, kv_dtype, seed=batch)
    expected = dense_attention(*exact, table, lengths)
    plan = DecodePlan(layout, table, lengths, split_tokens=256)
    assert plan._ragged_lengths and plan.launches(q.dtype, k.dtype) == 2
    hinted = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).clone()
    assert_parity(hinted.cpu().numpy(), expected, torch.float16)
    plan._ragged_lengths = False
    plain = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale)
    assert_parity(plain.cpu().numpy(), expected, torch.float16)
    torch.testing.assert_close(hinted, plain, rtol=1e-5, atol=1e-6)


def test_plan_derives_the_page_sharing_hint():
    """The plan streams K/V past the caches only when its table maps no page
    twice: the shared-prefix workload keeps them cacheable, the Llama-3-8B one
    streams, and a device-side CSR refresh falls back to cacheable."""
    shared = make_workload("ragged_shared_b16")
    plan = DecodePlan(shared.layout, shared.table, shared.lengths, split_tokens=shared.split_tokens)
    assert not plan._unshared_pages
    w = make_workload("llama3_8b_b4_l4096")
    plan = DecodePlan(w.layout, w.table, w.lengths, split_tokens=w.split_tokens)
    assert plan._unshared_pages
    aliased = w.table.copy()
    aliased[1, 0] = aliased[0, 0]                                  # one page now backs two sequences
    plan.refresh(aliased, w.lengths)
    assert not plan._unshared_pages
    plan.refresh(w.table, w.lengths)
    assert plan._unshared_pages
    indptr = torch.zeros(w.layout.batch + 1, dtype=torch.int32, device="cuda")
    indices = torch.zeros(1, dtype=torch.int32, device="cuda")
    last = torch.ones(w.layout.batch, dtype=torch.int32, device="cuda")
    plan.refresh_csr(indptr, indices, last)
    assert not plan._unshared_pages


def test_rejects_same_shape_noncontiguous_and_wrong_device():
    layout = Layout(1, 8, 2, 64, 16, 8)
    plan = DecodePlan(layout, np.arange(8, dtype=np.int32)[None], np.array([127]))
    q, k, v = make_tensors(layout)
    strided = torch.empty((1, 8, 128), device=q.device, dtype=q.dtype)[..., ::2]
    assert strided.shape == q.shape and not strided.is_contiguous()
    with pytest.raises(ValueError):
        plan.run(strided, k, v)
    with pytest.raises(ValueError):
        plan.run(q.cpu(), k, v)


# ---------------------------------------------------------------------------
# Beyond the reference matrix.


def test_golden_fixtures(golden_dir):
    from make_golden import SMALL_CASES, digest, small_case_inputs

    fixtures = np.load(golden_dir / "expected_outputs.npz")
    w = make_workload("fp32_b2_ragged")
    q, k, v = w.host_tensors()
    assert str(fixtures["fp32_b2_ragged/digest"]) == digest(q, k, v, w.table, w.lengths)
    cases = [("fp32_b2_ragged", w.layout, w.table, w.lengths, q, k, v, w.split_tokens)]
    for name in SMALL_CASES:
        layout, table, lengths, q, k, v = small_case_inputs(name)
        assert str(fixtures[f"{name}/digest"]) == digest(q, k, v, table, lengths)
        cases.append((name, layout, table, lengths, q, k, v, 17))
    for name, layout, table, lengths, q, k, v, split in cases:
        for merge in ("serial", "shared"):
            announce(f"golden {name} merge={merge}")
            plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
            tq, tk, tv = (torch.from_numpy(x).cuda() for x in (q, k, v))
            assert_parity(plan.run(tq, tk, tv).cpu().numpy(), fixtures[f"{name}/out"], q.dtype)


def test_nan_poisoned_workspace_live_states_written_dead_states_untouched():
    """initcheck analogue on a ragged batch with an empty sequence.

    Every state the merge reads -- partitions up to each sequence's end -- is
    written by the call; states past the end are never written (they keep the
    NaN poison) and never read (the output is finite and matches the oracle).
    This batch fills the device, so its workgroups combine their quarters: the
    slots of the folded quarters get the empty state (statistics written,
    l == 0) and their numerators, which no merge weights, stay untouched. Its
    grid is also large enough for the call to run over coarser partitions
    than the plan's (kernel_split): their states fill the workspace's leading
    part, laid out by that split, and the rest keeps the poison.
    """
    w = make_workload("ragged_shared_b16")
    layout = w.layout
    q, k, v = (torch.from_numpy(x).cuda() for x in w.host_tensors())
    for merge in ("serial", "shared"):
        plan = DecodePlan(layout, w.table, w.lengths, split_tokens=w.split_tokens, merge=merge)
        for t in (plan._numerator, plan._stats, plan._out):
            t.fill_(float("nan"))
        splits, split_tokens = plan.kernel_split(q.dtype)
        announce(f"nan-poison ragged_shared_b16 merge={merge}, kernel split {splits} x {split_tokens}")
        out = plan.run(q, k, v)
        torch.cuda.synchronize()
        assert torch.isfinite(out).all()
        assert_parity(out.cpu().numpy(), oracle(q, k, v, w.table, w.lengths), torch.float16)
        shape = (layout.batch, layout.query_heads, 4 * splits)
        used = int(np.prod(shape))
        num = plan._numerator.view(-1)[:used * layout.head_dim].view(*shape, layout.head_dim).cpu().numpy()
        st = plan._stats.view(-1)[:used * 2].view(*shape, 2).cpu().numpy()
        assert torch.isnan(plan._numerator.view(-1)[used * layout.head_dim:]).all()
        assert torch.isnan(plan._stats.view(-1)[used * 2:]).all()
        empty_slots = 0
        for b, length in enumerate(w.lengths):
            live = 4 * -(-int(length) // split_tokens)
            assert np.isfinite(st[b, :, :live]).all()
            holds = st[b, :, :live, 1] > 0                          # states with tokens
            assert np.isfinite(num[b, :, :live][holds]).all()
            empty = ~holds
            assert np.all(st[b, :, :live, 0][empty] == np.finfo(np.float32).min)
            empty_slots += int(empty.sum())
            assert np.isnan(num[b, :, live:]).all() and np.isnan(st[b, :, live:]).all()
        assert (w.lengths == 0).any() and empty_slots > 0


@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_refresh_loads_new_metadata_in_place(merge):
    """refresh(): new table and lengths, same buffers; graphs replay the new metadata.

    The captured launch keeps the host length bounds of its capture, so after a
    refresh it may run another (compacted) grid than an eager call: lengths
    past the captured bounds go to tail workgroups. Both match the FP64
    oracle, and each other to FP32 rounding."""
    layout = Layout(3, 16, 4, 128, 16, 3 * 64)
    rng = np.random.default_rng(11)
    q, k, v = make_tensors(layout, seed=11)
    table = rng.permutation(3 * 64).reshape(3, 64).astype(np.int32)
    lengths = np.array([1000, 17, 512], dtype=np.int32)
    plan = DecodePlan(layout, table, lengths, split_tokens=128, merge=merge, max_context=1024)
    assert plan.splits == 8 and plan.context_capacity == 1024 and plan.max_context == 1000
    announce(f"refresh merge={merge}")
    assert_parity(plan.run(q, k, v).cpu().numpy(), oracle(q, k, v, table, lengths), torch.float16)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            captured = plan.run(q, k, v)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    buffers = (plan._table.data_ptr(), plan._lengths.data_ptr(), plan._numerator.data_ptr())
    for new_lengths in ([1024, 0, 3], [0, 0, 0], [129, 1024, 700]):
        new_table = rng.permutation(3 * 64).reshape(3, 64).astype(np.int32)
        new_lengths = np.array(new_lengths, dtype=np.int32)
        plan.refresh(new_table, new_lengths)
        assert (plan._table.data_ptr(), plan._lengths.data_ptr(), plan._numerator.data_ptr()) == buffers
        assert plan.max_context == int(new_lengths.max())
        expected = oracle(q, k, v, new_table, new_lengths)
        eager = plan.run(q, k, v).clone()
        assert_parity(eager.cpu().numpy(), expected, torch.float16)
        captured.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert_parity(captured.cpu().numpy(), expected, torch.float16)
        torch.testing.assert_close(captured, eager, rtol=1e-5, atol=1e-6)


def test_refresh_rejects_what_does_not_fit():
    layout = Layout(2, 8, 2, 64, 16, 16)
    table = np.arange(16, dtype=np.int32).reshape(2, 8)
    plan = DecodePlan(layout, table, np.array([100, 60], dtype=np.int32), split_tokens=32)
    with pytest.raises(ValueError):
        plan.refresh(table, np.array([101, 0], dtype=np.int32))      # beyond the reserved context
    with pytest.raises(ValueError):
        plan.refresh(table[:, :4], np.array([10, 0], dtype=np.int32))  # table shape changed
    with pytest.raises(ValueError):
        plan.refresh(np.full((2, 8), 99, dtype=np.int32), np.array([10, 0], dtype=np.int32))  # live page out of range
    with pytest.raises(TypeError):
        plan.refresh(table.astype(np.float32), np.array([10, 0], dtype=np.int32))
    plan.refresh(table, np.array([100, 100], dtype=np.int32))
    assert plan.max_context == 100


def test_repeated_runs_are_bitwise_identical():
    w = make_workload("llama3_8b_b4_l4096")
    q, k, v = (torch.from_numpy(x).cuda() for x in w.host_tensors())
    for merge in ("serial", "shared"):
        announce(f"determinism merge={merge}")
        plan = DecodePlan(w.layout, w.table, w.lengths, split_tokens=w.split_tokens, merge=merge)
        first = plan.run(q, k, v).clone()
        for _ in range(5):
            torch.testing.assert_close(plan.run(q, k, v), first, rtol=0, atol=0)


def test_partial_then_merge_equals_decode():
    """The two stages called separately give the call's result. This launch
    combines quarters, and the separate merge reads every slot (empty states
    included) while the call merges the combined ones only: the same terms
    summed in another order, so equal to FP32 rounding, not bit for bit."""
    w = make_workload("llama3_8b_b4_l4096")
    q, k, v = (torch.from_numpy(x).cuda() for x in w.host_tensors())
    plan = DecodePlan(w.layout, w.table, w.lengths, split_tokens=w.split_tokens)
    full = plan.run(q, k, v).clone()
    plan._out.zero_()
    plan.run_partial(q, k, v)
    torch.testing.assert_close(plan.run_merge(), full, rtol=1e-5, atol=1e-6)


def test_raw_c_abi_matches_extension():
    """Calls the C ABI through ctypes with device pointers. ``pd_decode_ex`` given
    the plan's host bounds and hints plans the same launches as DecodePlan and
    gives the same bits; ``pd_decode`` (no bounds: plain grids, whose states
    may be combined differently) the same attention to FP32 rounding."""
    lib = cabi.load()
    w = make_workload("llama3_8b_b4_l4096")
    q, k, v = (torch.from_numpy(x).cuda() for x in w.host_tensors())
    plan = DecodePlan(w.layout, w.table, w.lengths, split_tokens=w.split_tokens)
    expected = plan.run(q, k, v).clone()
    table = torch.from_numpy(w.table).cuda()
    lengths = torch.from_numpy(w.lengths).cuda()
    numerator = torch.empty_like(plan._numerator)
    stats = torch.empty_like(plan._stats)
    out = torch.full_like(plan._out, float("nan"))
    L = w.layout
    stream = torch.cuda.current_stream().cuda_stream
    announce("raw C ABI pd_decode_ex with the plan's bounds and hints, then pd_decode")
    bounds = np.ascontiguousarray(w.lengths, dtype=np.int32)
    hints = (cabi.PD_HINT_UNSHARED_PAGES if plan._unshared_pages else 0) | \
        (cabi.PD_HINT_RAGGED_LENGTHS if plan._ragged_lengths else 0)
    for merge in (cabi.PD_MERGE_SERIAL, cabi.PD_MERGE_SHARED):
        out.fill_(float("nan"))
        status = lib.pd_decode_ex(q.data_ptr(), cabi.PD_DTYPE_F16, k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F16,
                                  1.0, 1.0, table.data_ptr(), lengths.data_ptr(), numerator.data_ptr(),
                                  stats.data_ptr(), out.data_ptr(), L.batch, L.query_heads, L.kv_heads,
                                  L.head_dim, L.page_size, w.table.shape[1], L.physical_pages, plan.splits,
                                  w.split_tokens, merge, hints, bounds.ctypes.data, ctypes.c_void_p(stream))
        assert status == cabi.PD_OK, cabi.status_string(lib, status)
        torch.cuda.synchronize()
        if merge == cabi.PD_MERGE_SERIAL:
            torch.testing.assert_close(out, expected, rtol=0, atol=0)
        else:
            torch.testing.assert_close(out, expected, rtol=0, atol=1e-6)
        out.fill_(float("nan"))
        status = lib.pd_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F16, table.data_ptr(),
                               lengths.data_ptr(), numerator.data_ptr(), stats.data_ptr(), out.data_ptr(),
                               L.batch, L.query_heads, L.kv_heads, L.head_dim, L.page_size, w.table.shape[1],
                               L.physical_pages, plan.splits, w.split_tokens, merge, ctypes.c_void_p(stream))
        assert status == cabi.PD_OK, cabi.status_string(lib, status)
        torch.cuda.synchronize()
        torch.testing.assert_close(out, expected, rtol=1e-5, atol=1e-6)


def test_device_page_guard_skips_invalid_ids():
    """Out-of-range page ids reaching the raw entry are skipped, never read."""
    lib = cabi.load()
    layout = Layout(2, 8, 2, 128, 16, 6)
    q, k, v = make_tensors(layout, dtype=torch.float32, seed=44)
    table = np.array([[0, 1, 1 << 30, 2], [3, -7, 4, 5]], dtype=np.int32)
    lengths = np.array([64, 50], dtype=np.int32)
    d_table = torch.from_numpy(table).cuda()
    d_lengths = torch.from_numpy(lengths).cuda()
    splits = 4
    numerator = torch.empty((2, 8, 4 * splits, 128), device="cuda")  # four states per partition
    stats = torch.empty((2, 8, 4 * splits, 2), device="cuda")
    out = torch.empty((2, 8, 128), device="cuda")
    announce("device page guard")
    status = lib.pd_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F32, d_table.data_ptr(),
                           d_lengths.data_ptr(), numerator.data_ptr(), stats.data_ptr(), out.data_ptr(),
                           2, 8, 2, 128, 16, 4, 6, splits, 16, 0,
                           ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert status == cabi.PD_OK
    torch.cuda.synchronize()
    qh, kh, vh = host(q, k, v)
    # Equivalent valid problem: drop the tokens of the invalid pages.
    keep = [[0, 1, 3], [0, 2, 3]]
    expected = np.zeros((2, 8, 128))
    for b in range(2):
        pos = [t for t in range(lengths[b]) if t // 16 in keep[b]]
        rows_k = np.stack([kh[table[b][t // 16], t % 16] for t in pos]).astype(np.float64)
        rows_v = np.stack([vh[table[b][t // 16], t % 16] for t in pos]).astype(np.float64)
        for h in range(8):
            s = rows_k[:, h // 4] @ qh[b, h].astype(np.float64) / np.sqrt(128)
            p = np.exp(s - s.max())
            expected[b, h] = p @ rows_v[:, h // 4] / p.sum()
    assert_parity(out.cpu().numpy(), expected, torch.float32)


def test_non_finite_free_inputs_with_uninitialised_padding_pages():
    """Pages no live token maps to may hold NaN; they must never reach the output."""
    layout = Layout(2, 8, 2, 64, 16, 8)
    q, k, v = make_tensors(layout, dtype=torch.float16, seed=45)
    table = np.array([[0, 1, -1, -1], [2, 3, 4, -1]], dtype=np.int32)
    lengths = np.array([20, 33], dtype=np.int32)
    for page in (5, 6, 7):
        k[page].fill_(float("nan"))
        v[page].fill_(float("inf"))
    # Slots past each sequence's end inside its last live page are unused too.
    k[1, 4:].fill_(float("nan"))
    v[1, 4:].fill_(float("nan"))
    k[4, 1:].fill_(float("inf"))
    v[4, 1:].fill_(float("nan"))
    for merge in ("serial", "shared"):
        announce(f"nan padding pages merge={merge}")
        plan = DecodePlan(layout, table, lengths, split_tokens=7, merge=merge)
        actual = plan.run(q, k, v).cpu().numpy()
        assert_parity(actual, oracle(q, k, v, table, lengths), torch.float16)
