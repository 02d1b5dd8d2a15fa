"""The C ABI's format, stage and append entries called directly through ctypes.

Device pointers and plain integers only, the way an FFI caller binds
``include/paged_decode.h``. Results are checked against the FP64 oracle
(attention) and the oracle's scatter (append, bit for bit).
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

KV_CODES = {torch.float8_e4m3fn: cabi.PD_DTYPE_FP8_E4M3, torch.float8_e5m2: cabi.PD_DTYPE_FP8_E5M2,
            torch.float16: cabi.PD_DTYPE_F16, torch.bfloat16: cabi.PD_DTYPE_BF16}


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def ragged_problem(layout, seed):
    rng = np.random.default_rng(seed)
    width = layout.physical_pages // layout.batch
    table = rng.permutation(layout.physical_pages).reshape(layout.batch, width).astype(np.int32)
    lengths = np.array([width * layout.page_size, 0, 37, width * layout.page_size - 5][:layout.batch], np.int32)
    return table, lengths


def quantize(layout, kv_dtype, seed):
    """bf16 q and K/V in kv_dtype with per-tensor scales, plus the exact float64 values."""
    q, k, v = host_tensors(layout, dtype=np.float32, seed=seed)
    qt = torch.from_numpy(q).to(torch.bfloat16)
    largest = float(torch.finfo(kv_dtype).max)
    k_scale, v_scale = float(np.abs(k).max()) / largest, float(np.abs(v).max()) / largest
    kt = (torch.from_numpy(k) / k_scale).to(kv_dtype)
    vt = (torch.from_numpy(v) / v_scale).to(kv_dtype)
    exact = (qt.double().numpy(), kt.double().numpy() * k_scale, vt.double().numpy() * v_scale)
    return (qt.cuda(), kt.cuda(), vt.cuda()), (k_scale, v_scale), exact


def workspace(layout, splits):
    shape = (layout.batch, layout.query_heads, 4 * splits)
    num = torch.full((*shape, layout.head_dim), float("nan"), device="cuda")
    stats = torch.full((*shape, 2), float("nan"), device="cuda")
    out = torch.full((layout.batch, layout.query_heads, layout.head_dim), float("nan"), device="cuda")
    return num, stats, out


@pytest.mark.parametrize("kv_dtype", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("merge", [cabi.PD_MERGE_SERIAL, cabi.PD_MERGE_SHARED])
def test_decode_ex_fp8_matches_oracle(kv_dtype, merge):
    announce(f"pd_decode_ex bf16 q, {kv_dtype} K/V, merge={merge}")
    lib = cabi.load()
    layout = Layout(4, 16, 4, 128, 16, 4 * 12)
    table, lengths = ragged_problem(layout, 3)
    (q, k, v), (k_scale, v_scale), exact = quantize(layout, kv_dtype, 21)
    split_tokens = 64
    splits = -(-int(lengths.max()) // split_tokens)
    num, stats, out = workspace(layout, splits)
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    status = lib.pd_decode_ex(q.data_ptr(), cabi.PD_DTYPE_BF16, k.data_ptr(), v.data_ptr(), KV_CODES[kv_dtype],
                              k_scale, v_scale, d_table.data_ptr(), d_lengths.data_ptr(), num.data_ptr(),
                              stats.data_ptr(), out.data_ptr(), layout.batch, layout.query_heads, layout.kv_heads,
                              layout.head_dim, layout.page_size, table.shape[1], layout.physical_pages, splits,
                              split_tokens, merge, cabi.PD_HINT_UNSHARED_PAGES, None, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    actual = out.cpu().numpy()
    assert_parity(actual, fp64.dense_attention(*exact, table, lengths), torch.bfloat16)
    np.testing.assert_array_equal(actual[1], 0.0)


@pytest.mark.parametrize("batch, pages_per_row, launches", [(2, 40, 2), (4, 9, 1)])
def test_partial_then_merge_entries_equal_decode_ex(batch, pages_per_row, launches):
    """pd_decode_partial_ex followed by pd_decode_merge gives pd_decode_ex's bits when
    pd_decode_ex makes the same two launches (rows of 1280 FP8 tokens at D64: 160 KB
    per KV head; a grid smaller than the device, whose partitions keep four states
    each, so that the merge reads the same states in the same order). Rows of 288
    tokens (36 KB) are one whole-row launch: the same attention to FP32 rounding,
    with the workspace left unwritten."""
    announce(f"pd_decode_partial_ex + pd_decode_merge, B{batch}, {pages_per_row} pages per row")
    lib = cabi.load()
    layout = Layout(batch, 32, 8, 64, 32, batch * pages_per_row)
    table, lengths = ragged_problem(layout, 8)
    (q, k, v), (k_scale, v_scale), exact = quantize(layout, torch.float8_e4m3fn, 5)
    split_tokens = 48
    splits = -(-int(lengths.max()) // split_tokens)
    args = (layout.batch, layout.query_heads, layout.kv_heads, layout.head_dim, layout.page_size, table.shape[1],
            layout.physical_pages, splits, split_tokens)
    assert cabi.launch_count(lib, cabi.PD_DTYPE_BF16, cabi.PD_DTYPE_FP8_E4M3, *args) == launches
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    num, stats, full = workspace(layout, splits)
    status = lib.pd_decode_ex(q.data_ptr(), cabi.PD_DTYPE_BF16, k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_FP8_E4M3,
                              k_scale, v_scale, d_table.data_ptr(), d_lengths.data_ptr(), num.data_ptr(),
                              stats.data_ptr(), full.data_ptr(), *args, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_NONE,
                              None, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    num2, stats2, staged = workspace(layout, splits)
    status = lib.pd_decode_partial_ex(q.data_ptr(), cabi.PD_DTYPE_BF16, k.data_ptr(), v.data_ptr(),
                                      cabi.PD_DTYPE_FP8_E4M3, k_scale, v_scale, d_table.data_ptr(),
                                      d_lengths.data_ptr(), num2.data_ptr(), stats2.data_ptr(), *args,
                                      cabi.PD_HINT_NONE, None, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    status = lib.pd_decode_merge(num2.data_ptr(), stats2.data_ptr(), staged.data_ptr(), d_lengths.data_ptr(),
                                 layout.batch, layout.query_heads, layout.head_dim, layout.page_size, table.shape[1],
                                 splits, split_tokens, cabi.PD_MERGE_SERIAL, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    if launches == 2:
        torch.testing.assert_close(staged, full, rtol=0, atol=0)
    else:
        torch.testing.assert_close(full, staged, rtol=2e-5, atol=2e-6)
        assert_parity(full.cpu().numpy(), fp64.dense_attention(*exact, table, lengths), torch.bfloat16)
        assert torch.isnan(num).all() and torch.isnan(stats).all()


@pytest.mark.parametrize("dtype", [torch.float8_e5m2, torch.bfloat16])
def test_append_entries_match_scatter(dtype):
    """pd_append_kv (explicit positions) and pd_append_kv_advance, bit for bit."""
    announce(f"pd_append_kv / pd_append_kv_advance {dtype}")
    lib = cabi.load()
    layout = Layout(3, 8, 2, 128, 16, 12)
    table = np.arange(12, dtype=np.int32).reshape(3, 4)[:, ::-1].copy()
    tokens = 2
    rng = np.random.default_rng(4)
    k_cache = torch.from_numpy(rng.standard_normal((12, 16, 2, 128)).astype(np.float32)).to(dtype).cuda()
    v_cache = torch.from_numpy(rng.standard_normal((12, 16, 2, 128)).astype(np.float32)).to(dtype).cuda()
    k_new = torch.from_numpy(rng.standard_normal((3, tokens, 2, 128)).astype(np.float32)).to(dtype).cuda()
    v_new = torch.from_numpy(rng.standard_normal((3, tokens, 2, 128)).astype(np.float32)).to(dtype).cuda()
    as_bytes = (lambda t: t.view(torch.uint8).cpu().numpy()) if dtype.itemsize == 1 else \
        (lambda t: t.view(torch.int16).cpu().numpy())
    d_table = torch.from_numpy(table).cuda()
    dims = (3, tokens, 2, 128, 16, 4, 12)

    positions = np.array([0, 17, 63], dtype=np.int32)  # the last sequence's second token is past the table
    expected_k = fp64.scatter_tokens(as_bytes(k_cache), table, positions, as_bytes(k_new))
    expected_v = fp64.scatter_tokens(as_bytes(v_cache), table, positions, as_bytes(v_new))
    d_positions = torch.from_numpy(positions).cuda()
    status = lib.pd_append_kv(k_new.data_ptr(), v_new.data_ptr(), KV_CODES[dtype], d_table.data_ptr(),
                              d_positions.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), *dims, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(as_bytes(k_cache), expected_k)
    np.testing.assert_array_equal(as_bytes(v_cache), expected_v)

    lengths = np.array([5, 62, 63], dtype=np.int32)  # the last sequence has no room for two tokens
    expected_k, grown = fp64.append_advance(as_bytes(k_cache), table, lengths, as_bytes(k_new))
    expected_v, _ = fp64.append_advance(as_bytes(v_cache), table, lengths, as_bytes(v_new))
    d_lengths = torch.from_numpy(lengths).cuda()
    status = lib.pd_append_kv_advance(k_new.data_ptr(), v_new.data_ptr(), KV_CODES[dtype], d_table.data_ptr(),
                                      d_lengths.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), *dims, 64,
                                      stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(as_bytes(k_cache), expected_k)
    np.testing.assert_array_equal(as_bytes(v_cache), expected_v)
    np.testing.assert_array_equal(d_lengths.cpu().numpy(), grown)
    assert grown.tolist() == [7, 64, 63]

    # A context capacity below the table's (what the caller's partitions
    # cover): sequence 0 grows 7 -> 9, the others would cross 9 and stay.
    expected_k, grown = fp64.append_advance(expected_k, table, grown, as_bytes(k_new), max_context=9)
    expected_v, _ = fp64.append_advance(expected_v, table, d_lengths.cpu().numpy(), as_bytes(v_new), max_context=9)
    status = lib.pd_append_kv_advance(k_new.data_ptr(), v_new.data_ptr(), KV_CODES[dtype], d_table.data_ptr(),
                                      d_lengths.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), *dims, 9,
                                      stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(as_bytes(k_cache), expected_k)
    np.testing.assert_array_equal(as_bytes(v_cache), expected_v)
    np.testing.assert_array_equal(d_lengths.cpu().numpy(), grown)
    assert grown.tolist() == [9, 64, 63]


def test_context_sharded_over_two_partial_launches():
    """The page-range sharding design on one GPU: two 'devices' each run the
    partition stage on their half of every sequence's pages, their states are
    concatenated (the all-gather), and one merge gives the unsharded result."""
    announce("context sharded over two partial launches")
    lib = cabi.load()
    layout = Layout(2, 8, 2, 128, 16, 2 * 64)
    rng = np.random.default_rng(12)
    table = rng.permutation(layout.physical_pages).reshape(2, 64).astype(np.int32)
    lengths = np.array([1024, 700], dtype=np.int32)
    q, k, v = (torch.from_numpy(x).cuda() for x in host_tensors(layout, dtype=np.float16, seed=6))
    split_tokens, half_pages = 128, 32
    half_tokens = half_pages * layout.page_size            # a multiple of split_tokens
    shard_splits = half_tokens // split_tokens
    dims = (layout.batch, layout.query_heads, layout.kv_heads, layout.head_dim, layout.page_size)
    states, stats = [], []
    for shard in range(2):
        sub_table = torch.from_numpy(np.ascontiguousarray(table[:, shard * half_pages:(shard + 1) * half_pages])).cuda()
        sub_lengths = torch.from_numpy(np.clip(lengths - shard * half_tokens, 0, half_tokens).astype(np.int32)).cuda()
        num, st, _ = workspace(layout, shard_splits)
        status = lib.pd_decode_partial(q.data_ptr(), k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F16,
                                       sub_table.data_ptr(), sub_lengths.data_ptr(), num.data_ptr(), st.data_ptr(),
                                       *dims, half_pages, layout.physical_pages, shard_splits, split_tokens, stream())
        assert status == cabi.PD_OK, cabi.status_string(lib, status)
        states.append(num)
        stats.append(st)
    # Shard 0 is full for every sequence, so the live states of the
    # concatenation are a prefix: exactly what the merge reads.
    num = torch.cat(states, dim=2).contiguous()
    st = torch.cat(stats, dim=2).contiguous()
    out = torch.full((layout.batch, layout.query_heads, layout.head_dim), float("nan"), device="cuda")
    d_lengths = torch.from_numpy(lengths).cuda()
    status = lib.pd_decode_merge(num.data_ptr(), st.data_ptr(), out.data_ptr(), d_lengths.data_ptr(),
                                 layout.batch, layout.query_heads, layout.head_dim, layout.page_size, table.shape[1],
                                 2 * shard_splits, split_tokens, cabi.PD_MERGE_SHARED, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    expected = fp64.dense_attention(*(t.cpu().numpy() for t in (q, k, v)), table, lengths)
    assert_parity(out.cpu().numpy(), expected, torch.float16)


@pytest.mark.parametrize("batch,query_heads,kv_heads,head_dim,stride", [
    (8, 16, 1, 64, 4), (8, 32, 4, 128, 2), (8, 48, 1, 128, 2), (8, 4, 1, 64, 1), (1, 16, 1, 64, 1),
    (8, 24, 6, 128, 2), (4, 40, 20, 64, 2), (8, 8, 2, 64, 2)])
def test_combined_quarter_states(batch, query_heads, kv_heads, head_dim, stride):
    """Workgroups holding several quarters of a partition store them combined.

    Four quarters of a full 16-head tile (MQA-like groups) and any two
    quarters become one state in the first quarter's slot, and the other slots
    get the empty state, when the launch fills the device (these grids have
    320-640 workgroups). pd_decode_partial + pd_decode_merge (which reads
    every slot) then agrees with pd_decode (which reads the combined slots
    only), and both match the oracle. stride 1: a shape that keeps four states
    per partition (four quarters of a 4-head tile), and a one-sequence grid
    smaller than the device. 6 KV heads make workgroups of 3 heads x 2
    quarters; 20 make five head groups of 4 per token row (streamed loads);
    2 KV heads at 320 8-wave workgroups take the 2-head x 2-quarter
    workgroups of mid-size grids.
    """
    announce(f"combined quarter states B{batch} Hq{query_heads}/Hkv{kv_heads} D{head_dim}")
    lib = cabi.load()
    width, page = 160, 16
    layout = Layout(batch, query_heads, kv_heads, head_dim, page, batch * width)
    rng = np.random.default_rng(17)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = np.array([width * page, 0, 37, width * page - 5, 600, 1, 513, 999][:batch], dtype=np.int32)
    for b, n in enumerate(lengths):
        table[b, (n + page - 1) // page:] = -1
    q, k, v = (torch.from_numpy(x).cuda() for x in host_tensors(layout, dtype=np.float16, seed=9))
    split_tokens = 64                                              # 16 tokens per quarter: every quarter holds a tile
    splits = -(-int(lengths.max()) // split_tokens)
    args = (layout.batch, query_heads, kv_heads, head_dim, layout.page_size, table.shape[1], layout.physical_pages,
            splits, split_tokens)
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    num, stats, fused = workspace(layout, splits)
    status = lib.pd_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F16, d_table.data_ptr(),
                           d_lengths.data_ptr(), num.data_ptr(), stats.data_ptr(), fused.data_ptr(), *args,
                           cabi.PD_MERGE_SERIAL, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    num2, stats2, staged = workspace(layout, splits)
    status = lib.pd_decode_partial(q.data_ptr(), k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F16, d_table.data_ptr(),
                                   d_lengths.data_ptr(), num2.data_ptr(), stats2.data_ptr(), *args, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    status = lib.pd_decode_merge(num2.data_ptr(), stats2.data_ptr(), staged.data_ptr(), d_lengths.data_ptr(),
                                 layout.batch, query_heads, head_dim, layout.page_size, table.shape[1], splits,
                                 split_tokens, cabi.PD_MERGE_SHARED, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    st = stats2.cpu().numpy()
    for b, length in enumerate(lengths):
        live = -(-int(length) // split_tokens)
        for s in range(live):
            slots = st[b, :, 4 * s:4 * s + 4]                      # [Hq, 4, (m, l)]
            assert np.all(slots[:, 0, 1] > 0)                      # the first quarter always holds tokens
            for quarter in range(4):
                if quarter % stride:
                    assert np.all(slots[:, quarter, 1] == 0.0)
                    assert np.all(slots[:, quarter, 0] == np.finfo(np.float32).min)
        if stride == 1 and int(length) >= split_tokens:
            assert np.all(st[b, :, 1, 1] > 0)                      # four separate states: quarter 1 holds tokens
        assert np.all(np.isnan(st[b, :, 4 * live:]))              # partitions past the end are never written
    expected = fp64.dense_attention(*(t.cpu().numpy() for t in (q, k, v)), table, lengths)
    assert_parity(fused.cpu().numpy(), expected, torch.float16)
    assert_parity(staged.cpu().numpy(), expected, torch.float16)
    torch.testing.assert_close(staged, fused, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("kv_heads,kv_dtype", [(8, torch.float16), (32, torch.float16), (8, torch.float8_e4m3fn)])
def test_page_sharing_hint_changes_no_bits(kv_heads, kv_dtype):
    """PD_HINT_UNSHARED_PAGES only changes how loads use the caches: on a
    batch whose sequences share prefix pages (so the hint is wrong), hinted
    and unhinted calls give the same bits, for the 2-group (8 KV heads) and
    4+-group (32 KV heads) streaming choices and FP8."""
    announce(f"page-sharing hint Hkv{kv_heads} {kv_dtype}")
    lib = cabi.load()
    batch, width, page = 16, 32, 16
    layout = Layout(batch, 32, kv_heads, 128, page, batch * width)
    rng = np.random.default_rng(3)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    table[1:, :8] = table[0, :8]                                   # an 8-page prefix shared by every sequence
    lengths = rng.integers(129, width * page + 1, size=batch).astype(np.int32)
    for b, n in enumerate(lengths):
        table[b, (n + page - 1) // page:] = -1
    if kv_dtype == torch.float16:
        q, k, v = (torch.from_numpy(x).cuda() for x in host_tensors(layout, dtype=np.float16, seed=2))
        codes, scales = (cabi.PD_DTYPE_F16, cabi.PD_DTYPE_F16), (1.0, 1.0)
    else:
        (q, k, v), scales, _ = quantize(layout, kv_dtype, 2)
        codes = (cabi.PD_DTYPE_BF16, KV_CODES[kv_dtype])
    split_tokens = 64
    splits = -(-int(lengths.max()) // split_tokens)
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    outs = []
    for hint in (cabi.PD_HINT_NONE, cabi.PD_HINT_UNSHARED_PAGES):
        num, stats, out = workspace(layout, splits)
        status = lib.pd_decode_ex(q.data_ptr(), codes[0], k.data_ptr(), v.data_ptr(), codes[1], *scales,
                                  d_table.data_ptr(), d_lengths.data_ptr(), num.data_ptr(), stats.data_ptr(),
                                  out.data_ptr(), batch, 32, kv_heads, 128, page, width, layout.physical_pages,
                                  splits, split_tokens, cabi.PD_MERGE_SERIAL, hint, None, stream())
        assert status == cabi.PD_OK, cabi.status_string(lib, status)
        outs.append(out)
    torch.cuda.synchronize()
    torch.testing.assert_close(outs[1], outs[0], rtol=0, atol=0)
    assert torch.isfinite(outs[0]).all()


def int32_array(values):
    return np.ascontiguousarray(values, dtype=np.int32)


BOUND_CASES = {
    # name: (layout args (B, Hq, Hkv, D, T, pages per sequence), lengths, split_tokens, dtype)
    "gqa_ragged": ((4, 32, 8, 128, 16, 64), [1024, 0, 517, 1000], 64, np.float16),
    "mqa_combined_tail": ((64, 16, 1, 64, 16, 64), None, 64, np.float16),
    "mid_grid_combined_tail": ((16, 32, 8, 128, 16, 256), [4096, 4000, 2500, 4096, 4096, 3000, 4096, 1] * 2, 256,
                               np.float16),
    "fp32": ((2, 8, 2, 64, 16, 16), [100, 256], 32, np.float32),
}


@pytest.mark.parametrize("bounds_kind", ["exact", "half", "zero", "above"])
@pytest.mark.parametrize("case", sorted(BOUND_CASES))
def test_length_bounds_compact_the_grid_without_changing_results(case, bounds_kind):
    """Host length bounds (pd_decode_ex's length_bounds) only reshape the grid:
    exact bounds drop the partitions past each sequence's end; bounds below
    the device lengths ("half", "zero") put the later partitions on the tail
    workgroups, which stride over them (with the quarter combine in the MQA
    and mid-grid cases, so the combine slots are reused across partitions);
    bounds above them change nothing. Every variant matches the FP64 oracle
    and the unbounded call to FP32 rounding."""
    (b, hq, hkv, d, t, per_seq), lengths, split_tokens, dtype = BOUND_CASES[case]
    announce(f"length bounds {case} {bounds_kind}")
    lib = cabi.load()
    layout = Layout(b, hq, hkv, d, t, b * per_seq)
    rng = np.random.default_rng(41)
    table = rng.permutation(layout.physical_pages).reshape(b, per_seq).astype(np.int32)
    if lengths is None:
        lengths = rng.integers(0, per_seq * t + 1, size=b)
        lengths[0] = per_seq * t
    lengths = int32_array(lengths)
    bounds = {"exact": lengths, "half": lengths // 2, "zero": np.zeros_like(lengths),
              "above": np.minimum(lengths + 3 * split_tokens, per_seq * t)}[bounds_kind]
    bounds = int32_array(bounds)
    host = host_tensors(layout, dtype=dtype, seed=9)
    q, k, v = (torch.from_numpy(x).cuda() for x in host)
    code = cabi.PD_DTYPE_F32 if dtype == np.float32 else cabi.PD_DTYPE_F16
    splits = -(-int(lengths.max()) // split_tokens)
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    outs = []
    for bound_ptr in (None, bounds.ctypes.data_as(ctypes.c_void_p)):
        num, stats, out = workspace(layout, splits)
        status = lib.pd_decode_ex(q.data_ptr(), code, k.data_ptr(), v.data_ptr(), code, 1.0, 1.0,
                                  d_table.data_ptr(), d_lengths.data_ptr(), num.data_ptr(), stats.data_ptr(),
                                  out.data_ptr(), b, hq, hkv, d, t, per_seq, layout.physical_pages, splits,
                                  split_tokens, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_UNSHARED_PAGES, bound_ptr,
                                  stream())
        assert status == cabi.PD_OK, cabi.status_string(lib, status)
        outs.append(out)
    torch.cuda.synchronize()
    expected = fp64.dense_attention(*host, table, lengths)
    for out in outs:
        assert_parity(out.cpu().numpy(), expected, dtype)
    torch.testing.assert_close(outs[1], outs[0], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(outs[1].cpu().numpy()[lengths == 0], 0.0)


def test_length_bounds_partition_stage_writes_every_live_state():
    """pd_decode_partial_ex with bounds far below the device lengths still writes
    every live state (tail workgroups cover them) and none past each sequence's
    end: NaN-poisoned slots past the end stay NaN, and pd_decode_merge over the
    workspace matches the FP64 oracle."""
    announce("length bounds: partition stage coverage")
    lib = cabi.load()
    layout = Layout(3, 16, 4, 128, 16, 3 * 32)
    rng = np.random.default_rng(5)
    table = rng.permutation(layout.physical_pages).reshape(3, 32).astype(np.int32)
    lengths = int32_array([512, 77, 300])
    bounds = int32_array([16, 0, 100])
    host = host_tensors(layout, dtype=np.float16, seed=4)
    q, k, v = (torch.from_numpy(x).cuda() for x in host)
    split_tokens = 32
    splits = 16
    num, stats, out = workspace(layout, splits)
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    dims = (3, 16, 4, 128, 16, 32, layout.physical_pages, splits, split_tokens)
    status = lib.pd_decode_partial_ex(q.data_ptr(), cabi.PD_DTYPE_F16, k.data_ptr(), v.data_ptr(), cabi.PD_DTYPE_F16,
                                      1.0, 1.0, d_table.data_ptr(), d_lengths.data_ptr(), num.data_ptr(),
                                      stats.data_ptr(), *dims, cabi.PD_HINT_NONE,
                                      bounds.ctypes.data_as(ctypes.c_void_p), stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    status = lib.pd_decode_merge(num.data_ptr(), stats.data_ptr(), out.data_ptr(), d_lengths.data_ptr(), 3, 16, 128,
                                 16, 32, splits, split_tokens, cabi.PD_MERGE_SERIAL, stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    torch.cuda.synchronize()
    st = stats.cpu().numpy()
    for b, n in enumerate(lengths):
        live_states = 4 * (-(-int(n) // split_tokens))
        assert np.isfinite(st[b, :, :live_states]).all()
        assert np.isnan(st[b, :, live_states:]).all()
    assert_parity(out.cpu().numpy(), fp64.dense_attention(*host, table, lengths), np.float16)


@pytest.mark.parametrize("kv_dtype", [torch.float16, torch.float8_e4m3fn])
def test_lengths_past_the_callers_partitions_are_not_read(kv_dtype):
    """Device lengths above splits * split_tokens (but inside the table): the
    caller's partitions end there, and so does the attention, as in the
    reference's grid of `splits` partitions (decode.cu:42-44, :176). With
    host bounds the full call runs over a coarser split (2 x 512 for the
    caller's 3 x 256) whose last partition would reach further; it must give
    the same result as the call without bounds and as the FP64 oracle over
    the first 768 tokens of every sequence."""
    announce(f"lengths past the caller's partitions, {kv_dtype}")
    lib = cabi.load()
    batch, per_seq, split_tokens, splits = 64, 64, 256, 3
    layout = Layout(batch, 32, 8, 128, 16, batch * per_seq)
    rng = np.random.default_rng(19)
    table = rng.permutation(layout.physical_pages).reshape(batch, per_seq).astype(np.int32)
    lengths = int32_array(np.full(batch, 1000))
    lengths[::7] = rng.integers(700, 1025, size=len(lengths[::7]))
    bounds = int32_array(lengths)
    assert cabi.kernel_split(lib, cabi.PD_DTYPE_F16, KV_CODES[kv_dtype], batch, 32, 8, 128, 16, per_seq,
                             layout.physical_pages, splits, split_tokens, bounds, 256) == (2, 512)
    if kv_dtype == torch.float16:
        host = host_tensors(layout, dtype=np.float16, seed=12)
        q, k, v = (torch.from_numpy(x).cuda() for x in host)
        codes, scales = (cabi.PD_DTYPE_F16, cabi.PD_DTYPE_F16), (1.0, 1.0)
    else:
        (q, k, v), scales, host = quantize(layout, kv_dtype, 12)
        codes = (cabi.PD_DTYPE_BF16, KV_CODES[kv_dtype])
    d_table, d_lengths = torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()
    outs = []
    for bound_ptr in (None, bounds.ctypes.data_as(ctypes.c_void_p)):
        num, stats, out = workspace(layout, splits)
        status = lib.pd_decode_ex(q.data_ptr(), codes[0], k.data_ptr(), v.data_ptr(), codes[1], *scales,
                                  d_table.data_ptr(), d_lengths.data_ptr(), num.data_ptr(), stats.data_ptr(),
                                  out.data_ptr(), batch, 32, 8, 128, 16, per_seq, layout.physical_pages, splits,
                                  split_tokens, cabi.PD_MERGE_SERIAL, cabi.PD_HINT_UNSHARED_PAGES, bound_ptr,
                                  stream())
        assert status == cabi.PD_OK, cabi.status_string(lib, status)
        outs.append(out)
    torch.cuda.synchronize()
    expected = fp64.dense_attention(*host, table, np.minimum(lengths, splits * split_tokens))
    for out in outs:
        assert_parity(out.cpu().numpy(), expected, np.float16)
    torch.testing.assert_close(outs[1], outs[0], rtol=1e-5, atol=1e-6)


def test_stream_read_reads_without_writing():
    """The streaming-read ceiling kernel reads whole and partial blocks of both
    buffers and leaves its sink untouched (zeros fold to zero, never the magic
    value), also inside a captured graph."""
    announce("pd_stream_read")
    lib = cabi.load()
    a = torch.zeros(3 * 2048 * 4 + 4, dtype=torch.int32, device="cuda")   # 3 blocks + one vector
    b = torch.zeros(5 * 4, dtype=torch.int32, device="cuda")             # less than a block
    sink = torch.full((2,), 7, dtype=torch.int32, device="cuda")
    status = lib.pd_stream_read(a.data_ptr(), a.numel() * 4, b.data_ptr(), b.numel() * 4, sink.data_ptr(), stream())
    assert status == cabi.PD_OK, cabi.status_string(lib, status)
    from paged_decode.runtime import load_extension

    ext = load_extension()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            ext.stream_read(a, b, a.numel() * 4, 64, sink)
    for _ in range(3):
        graph.replay()
    torch.cuda.synchronize()
    assert sink.tolist() == [7, 7]
    with pytest.raises(RuntimeError, match="fit"):
        ext.stream_read(a, b, a.numel() * 4 + 16, 0, sink)
