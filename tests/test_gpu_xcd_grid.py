"""Full decode calls on the XCD-grouped partition grid.

A plain rectangular call whose host bounds give every sequence the same
partitions runs its partition workgroups so that each row group (a
sequence's head group) stays on one XCD, and its merge workgroups so that
each row is merged on that same XCD (``plan_xcd``, ``block_coords``,
``merge_xcd_row``). With eight head groups per sequence (the MHA shape here)
the plain grids already keep row groups on one XCD, and only the merge is
XCD-grouped. The planner's choice for these shapes, and that both
mappings cover every state and row exactly once on matching XCDs, is checked
on the CPU by the address audit (``tests/address_audit.cpp``, problems named
``xcd ...``). Here the calls are checked against the FP64 oracle on exactly the
values the device holds, for FP16, BF16, FP8 and FP32, both merges, and both
merge kernels (one row per workgroup, and one wave per row); and against the
same call without bounds, whose plain grids give the same attention to FP32
rounding. Two calls in a row must agree bit for bit.
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

# name: (batch, query heads, KV heads, head_dim, page, length, split_tokens, formats)
# The names match the address audit's "xcd ..." problems.
SHAPES = {
    "gqa4 B8 Hq32/8 D128 L1024 split 128": (8, 32, 8, 128, 16, 1024, 128, ("f16", "bf16", "e4m3")),
    "mqa B64 Hq16/1 D64 L1024 split 256": (64, 16, 1, 64, 16, 1024, 256, ("f16", "e4m3")),
    "mha B2 Hq16/16 D128 L2048 split 256": (2, 16, 16, 128, 16, 2048, 256, ("f16",)),
    "fp32 B8 Hq16/8 D64 L1024 split 128": (8, 16, 8, 64, 16, 1024, 128, ("f32",)),
}
DTYPES = {
    "f16": (torch.float16, None),
    "bf16": (torch.bfloat16, None),
    "e4m3": (torch.float16, torch.float8_e4m3fn),
    "f32": (torch.float32, None),
}
CASES = [(name, fmt) for name, shape in SHAPES.items() for fmt in shape[-1]]


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


@pytest.mark.parametrize("merge", ["serial", "shared"])
@pytest.mark.parametrize("name,fmt", CASES)
def test_xcd_grouped_calls_match_oracle_and_plain_grids(name, fmt, merge):
    batch, heads, kv_heads, dim, page, length, split, _ = SHAPES[name]
    q_dtype, kv_dtype = DTYPES[fmt]
    announce(f"xcd-grouped call {name} {fmt} merge={merge}")
    width = length // page
    rng = np.random.default_rng(batch + heads)
    layout = Layout(batch, heads, kv_heads, dim, page, batch * width)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = np.full(batch, length, dtype=np.int32)
    (q, k, v), (k_scale, v_scale), exact = device_inputs(layout, q_dtype, kv_dtype, seed=batch)
    plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
    assert plan.kernel_split(q.dtype, k.dtype) == (plan.splits, split)  # no coarser partitions here
    plan._numerator.fill_(float("nan"))
    plan._stats.fill_(float("nan"))
    outs = []
    for _ in range(2):  # a second call reads what the first left in the XCDs' caches
        outs.append(plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).clone())
    torch.cuda.synchronize()
    torch.testing.assert_close(outs[1], outs[0], rtol=0, atol=0)
    actual = outs[0].cpu().numpy()
    assert_parity(actual, fp64.dense_attention(*exact, table, lengths), q_dtype)
    # Without bounds the same entry plans plain partition grids (and, but for
    # the MHA shape, plain merge grids).
    out = torch.empty_like(outs[0])
    plan._extension.decode(q, k, v, plan._table, plan._lengths, plan._numerator, plan._stats, out, split,
                           int(plan.merge_implementation == "shared"), k_scale, v_scale)
    torch.testing.assert_close(out, outs[0], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("merge", ["serial", "shared"])
@pytest.mark.parametrize("name,fmt", [("gqa4 B8 Hq32/8 D128 L1024 split 128", "f16"),
                                      ("mqa B64 Hq16/1 D64 L1024 split 256", "e4m3"),
                                      ("fp32 B8 Hq16/8 D64 L1024 split 128", "f32")])
def test_xcd_grouped_calls_with_tail_items(name, fmt, merge):
    """Reserved context: the plan's bounds (its host lengths) reach half of
    max_context, so the grid carries tail items, which follow each row group's
    main items on its XCD. The device lengths then grow past the bounds to the
    whole reserve, as appends on the device would, and the tail items cover
    the growth."""
    batch, heads, kv_heads, dim, page, length, split, _ = SHAPES[name]
    q_dtype, kv_dtype = DTYPES[fmt]
    announce(f"xcd-grouped call with tail items {name} {fmt} merge={merge}")
    width = length // page
    rng = np.random.default_rng(batch + heads + 1)
    layout = Layout(batch, heads, kv_heads, dim, page, batch * width)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = np.full(batch, length // 2, dtype=np.int32)
    (q, k, v), (k_scale, v_scale), exact = device_inputs(layout, q_dtype, kv_dtype, seed=batch + 1)
    plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge, max_context=length)
    for live in (length // 2, length - 1, length):
        plan._lengths.fill_(live)  # as device-side appends would; the host bounds stay at length // 2
        out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).clone()
        torch.cuda.synchronize()
        grown = np.full(batch, live, dtype=np.int32)
        assert_parity(out.cpu().numpy(), fp64.dense_attention(*exact, table, grown), q_dtype)


def stress_cases(count=32, seed=2026):
    """Seeded shapes for the stress below (kept small enough for the FP64 oracle)."""
    rng = np.random.default_rng(seed)
    layouts = [(32, 8), (16, 8), (32, 4), (16, 2), (16, 1), (32, 32), (8, 8), (64, 8), (24, 8)]
    formats = ["f16", "bf16", "e4m3", "f32"]
    cases = []
    for _ in range(count):
        heads, kv_heads = layouts[rng.integers(len(layouts))]
        batch = int(rng.choice([1, 2, 3, 4, 6, 8, 16] if kv_heads < 32 else [1, 2]))
        cases.append(dict(heads=heads, kv_heads=kv_heads, batch=batch, fmt=formats[rng.integers(len(formats))],
                          dim=int(rng.choice([64, 128])), page=int(rng.choice([16, 32])),
                          split=int(rng.choice([64, 128, 256])), length=int(rng.integers(1, 1025)),
                          reserve=int(rng.choice([1, 2])), merge="shared" if rng.random() < 0.5 else "serial"))
    return cases


def test_randomized_uniform_calls():
    """A seeded stress over uniform batches with host bounds: batch sizes and
    head layouts that do and do not make the XCD-grouped grid (sequences x head
    groups a multiple of 8 or not, eight head groups per sequence or fewer),
    reserved context (tail rows) or none, page 16 / 32, D 64 / 128, FP16, BF16,
    FP8 and FP32, both merges; every call against the FP64 oracle."""
    for case, c in enumerate(stress_cases()):
        announce(f"xcd stress {case}: {c}")
        q_dtype, kv_dtype = DTYPES[c["fmt"]]
        batch, length, page = c["batch"], c["length"], c["page"]
        width = -(-length * c["reserve"] // page)
        layout = Layout(batch, c["heads"], c["kv_heads"], c["dim"], page, batch * width)
        table = np.random.default_rng(case).permutation(batch * width).reshape(batch, width).astype(np.int32)
        lengths = np.full(batch, length, dtype=np.int32)
        (q, k, v), (k_scale, v_scale), exact = device_inputs(layout, q_dtype, kv_dtype, seed=case)
        plan = DecodePlan(layout, table, lengths, split_tokens=c["split"], merge=c["merge"],
                          max_context=length * c["reserve"])
        out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).clone()
        torch.cuda.synchronize()
        assert_parity(out.cpu().numpy(), fp64.dense_attention(*exact, table, lengths), q_dtype)
