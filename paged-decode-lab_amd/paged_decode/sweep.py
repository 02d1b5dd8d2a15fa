"""Named shape sweeps over the launch planner's rules (``bench.py --sweep``).

Each list holds the shapes one group of planner rules was decided on
(``csrc/partition_map.h``: ``plan_items``, ``coarse_split``, ``plan_mfma``,
``plan_xcd``, ``plan_rows``; ``csrc/merge_map.h``: ``plan_merge``). A sweep
times every shape as full decode calls (one hipGraph of K calls, K/V rotated
over >= 2 GiB of buffer sets so no call is served from the Infinity Cache), the
partition launch alone, and optionally the staged path (partition + merge
entries) at forced kernel splits: the caller's split times c for each c of
``coarse``. Each shape prints one JSON line with the per-call times and the
plan the library chose (``DecodePlan.launch_plan``), so a rule change can be
checked against every shape its comment cites with one command, run before
and after the change.

K/V values are drawn on the device (seeded N(0,1)): the sweep measures
launches; parity lives in the GPU tests.
"""
from dataclasses import dataclass
import json
import math
import sys

import numpy as np

from .layout import Layout
from .workload import make_metadata, make_workload

ROTATION_BYTES = 2 << 30


@dataclass(frozen=True)
class Shape:
    name: str
    batch: int
    query_heads: int
    kv_heads: int
    head_dim: int
    page_size: int
    lengths: str          # "uniform:L" | "ragged:L" (U[0, L] seeded, one empty) | "skewed:L" (one at L, the
                          # rest U[0, L/2]) | "reference:L" (make_metadata seed 123) | "workload:NAME" (a named
                          # workload's own table and lengths)
    split_tokens: int
    fmt: str = "f16"      # f16 | bf16 | fp8 (e4m3 K/V under an f16 q) | f32
    reserve: int = 1      # max_context = reserve x the longest sequence
    shared_prefix: float = 0.0  # leading fraction of the longest sequence's pages, mapped to one shared set
    coarse: tuple = ()    # kernel split factors c timed through the stage entries
    bounds: bool = True   # False: calls without host length bounds (the library sees device lengths only)
    runs: bool = True     # False: calls without shared-prefix runs (every sequence reads its own pages)


def _s(name, b, hq, hkv, d, t, lengths, split, **kw):
    return Shape(name, b, hq, hkv, d, t, lengths, split, **kw)


# Coarser partitions for full calls on large grids (coarse_split).
COARSE = [
    _s("ragged+shared B16 T32 split 128", 16, 32, 8, 128, 32, "workload:ragged_shared_b16", 128,
       coarse=(1, 2, 4, 8)),
    _s("reference B16 L4096 split 256", 16, 32, 8, 128, 16, "reference:4096", 256, coarse=(1, 2, 4)),
    _s("uniform B16 L4096 split 256", 16, 32, 8, 128, 16, "uniform:4096", 256, coarse=(1, 2, 4)),
    _s("uniform B32 L4096 split 256", 32, 32, 8, 128, 16, "uniform:4096", 256, coarse=(1, 2, 4)),
    _s("uniform B64 L2048 split 256", 64, 32, 8, 128, 16, "uniform:2048", 256, coarse=(1, 2, 4)),
    _s("fp8 B16 L4096 split 256", 16, 32, 8, 128, 16, "uniform:4096", 256, fmt="fp8", coarse=(1, 2, 4, 8)),
    _s("fp8 B64 L2048 split 256", 64, 32, 8, 128, 16, "uniform:2048", 256, fmt="fp8", coarse=(1, 2, 4, 8)),
    _s("mqa B512 L1024 D64 split 256", 512, 16, 1, 64, 16, "uniform:1024", 256, coarse=(1, 2, 4, 8)),
    _s("long mha B1 L32768 split 128", 1, 32, 32, 128, 16, "uniform:32768", 128, coarse=(1, 2, 4, 8)),
    _s("llama3-8b B4 L4096 split 256", 4, 32, 8, 128, 16, "uniform:4096", 256, coarse=(1, 2, 4)),
    _s("llama3-8b fp8 B4 L4096 split 256", 4, 32, 8, 128, 16, "uniform:4096", 256, fmt="fp8", coarse=(1, 2)),
    _s("mqa B128 L1024 D64 split 256", 128, 16, 1, 64, 16, "uniform:1024", 256, coarse=(1, 2, 4)),
    _s("reference B4 L4096 split 256", 4, 32, 8, 128, 16, "reference:4096", 256, coarse=(1, 2)),
]

# Reserved context (max_context above the longest sequence): tail items and
# work lists under host bounds (plan_items), against calls without bounds.
RESERVED = [
    _s(f"{base} reserve x{r}{'' if bounds else ' no bounds'}", *args, reserve=r, bounds=bounds, **kw)
    for base, args, kw in [
        ("llama3-8b B4 L4096", (4, 32, 8, 128, 16, "uniform:4096", 256), {}),
        ("reference B4 L4096", (4, 32, 8, 128, 16, "reference:4096", 256), {}),
        ("uniform B32 L4096", (32, 32, 8, 128, 16, "uniform:4096", 256), {}),
        ("ragged+shared B16 T32 split 128", (16, 32, 8, 128, 32, "workload:ragged_shared_b16", 128), {}),
    ]
    for r in (1, 2, 4) for bounds in (True, False)
]

# Small grids (dispatch_mfma: smaller workgroups when 8-wave ones leave CUs idle).
SMALL = [
    _s("B1 L4096", 1, 32, 8, 128, 16, "uniform:4096", 256),
    _s("B1 L2048", 1, 32, 8, 128, 16, "uniform:2048", 256),
    _s("fp8 B1 L4096", 1, 32, 8, 128, 16, "uniform:4096", 256, fmt="fp8"),
    _s("B2 L4096", 2, 32, 8, 128, 16, "uniform:4096", 256),
    _s("B1 L8192", 1, 32, 8, 128, 16, "uniform:8192", 256),
    _s("B3 L4096", 3, 32, 8, 128, 16, "uniform:4096", 256),
    _s("B1 L4096 Hkv4", 1, 32, 4, 128, 16, "uniform:4096", 256),
    _s("mqa B4 L1024 D64", 4, 16, 1, 64, 16, "uniform:1024", 256),
    _s("reference B1 L4096", 1, 32, 8, 128, 16, "reference:4096", 256),
]

# Mid-size grids (2 KV heads x 2 quarters per 4-wave workgroup) and the
# ragged-lengths hint.
MID = [
    _s("B8 L4096", 8, 32, 8, 128, 16, "uniform:4096", 256),
    _s("B16 L4096 Hq16/Hkv2", 16, 16, 2, 128, 16, "uniform:4096", 256),
    _s("B8 L4096 Hq32/Hkv4", 8, 32, 4, 128, 16, "uniform:4096", 256),
    _s("B16 ragged L4096", 16, 32, 8, 128, 16, "ragged:4096", 256),
    _s("B32 ragged L4096", 32, 32, 8, 128, 16, "ragged:4096", 256),
    _s("B32 ragged L8192", 32, 32, 8, 128, 16, "ragged:8192", 256),
    _s("fp8 B16 ragged L4096", 16, 32, 8, 128, 16, "ragged:4096", 256, fmt="fp8"),
    _s("fp8 B32 ragged L4096", 32, 32, 8, 128, 16, "ragged:4096", 256, fmt="fp8"),
]

# XCD-grouped partition and merge grids (plan_xcd).
XCD = [
    _s("B6 L4096", 6, 32, 8, 128, 16, "uniform:4096", 256),
    _s("B4 L4096 D64", 4, 32, 8, 64, 16, "uniform:4096", 256),
    _s("B4 L4096 T32", 4, 32, 8, 128, 32, "uniform:4096", 256),
    _s("B4 L4096 Hq64/Hkv4", 4, 64, 4, 128, 16, "uniform:4096", 256),
    _s("B8 L4096 Hkv2 GQA16", 8, 32, 2, 128, 16, "uniform:4096", 256),
    _s("B16 L2048 Hq16/Hkv1 D128", 16, 16, 1, 128, 16, "uniform:2048", 256),
    _s("fp32 B4 L4096", 4, 32, 8, 128, 16, "uniform:4096", 256, fmt="f32"),
    _s("fp8 B8 L4096", 8, 32, 8, 128, 16, "uniform:4096", 256, fmt="fp8"),
    _s("mha B2 L8192 Hkv32", 2, 32, 32, 128, 16, "uniform:8192", 256),
    _s("B64 L1024", 64, 32, 8, 128, 16, "uniform:1024", 256),
    _s("ragged B8 L4096", 8, 32, 8, 128, 16, "ragged:4096", 256),
]

# Whole-row launches (plan_rows: rows of at most 128 KB of K and V), against
# the two-launch path through the stage entries (coarse factor 1).
ROWS = [
    _s("fp32 B2 L256 Hq8/Hkv2 D64", 2, 8, 2, 64, 16, "uniform:256", 256, fmt="f32", coarse=(1,)),
    _s("B4 L256", 4, 32, 8, 128, 16, "uniform:256", 256, coarse=(1,)),
    _s("B16 L256", 16, 32, 8, 128, 16, "uniform:256", 256, coarse=(1,)),
    _s("B32 L256 split 128", 32, 32, 8, 128, 16, "uniform:256", 128, coarse=(1,)),
    _s("B64 L128 split 64", 64, 32, 8, 128, 16, "uniform:128", 64, coarse=(1,)),
    _s("mqa B128 L512 D64", 128, 16, 1, 64, 16, "uniform:512", 256, coarse=(1,)),
    _s("mqa B256 L256 D64", 256, 16, 1, 64, 16, "uniform:256", 256, coarse=(1,)),
]

# Shared prefixes (plan_prefix_items): work lists whose partitions inside
# several sequences' common prefix are scored once for up to 16 / GT of them,
# against the same calls without runs (one read per sequence).
PREFIX = [
    _s(f"{base}{'' if runs else ' no runs'}", *args, runs=runs, **kw)
    for base, args, kw in [
        ("ragged+shared B16 T32 split 128", (16, 32, 8, 128, 32, "workload:ragged_shared_b16", 128), {}),
        ("skewed B16 L8192 T32 50% shared", (16, 32, 8, 128, 32, "skewed:8192", 128), {"shared_prefix": 0.5}),
        ("skewed B32 L4096 25% shared", (32, 32, 8, 128, 16, "skewed:4096", 256), {"shared_prefix": 0.25}),
        ("fp8 skewed B16 L8192 T32 25% shared", (16, 32, 8, 128, 32, "skewed:8192", 128),
         {"shared_prefix": 0.25, "fmt": "fp8"}),
        ("mha skewed B16 Hq16/16 L4096 25% shared", (16, 16, 16, 128, 16, "skewed:4096", 256),
         {"shared_prefix": 0.25}),
        ("gqa8 skewed B16 Hq32/4 L4096 25% shared", (16, 32, 4, 128, 16, "skewed:4096", 256),
         {"shared_prefix": 0.25}),
        # Several samples of one prompt (equal lengths): a rectangular grid that
        # becomes a work list when the items remove enough of it.
        ("samples B16 L4096 50% shared", (16, 32, 8, 128, 16, "uniform:4096", 256), {"shared_prefix": 0.5}),
        ("samples B16 L4096 25% shared", (16, 32, 8, 128, 16, "uniform:4096", 256), {"shared_prefix": 0.25}),
        ("samples B16 L4096 12.5% shared", (16, 32, 8, 128, 16, "uniform:4096", 256), {"shared_prefix": 0.125}),
        ("samples B8 L8192 50% shared", (8, 32, 8, 128, 16, "uniform:8192", 256), {"shared_prefix": 0.5}),
        ("samples B32 L2048 50% shared", (32, 32, 8, 128, 16, "uniform:2048", 256), {"shared_prefix": 0.5}),
        ("samples B32 L4096 50% shared", (32, 32, 8, 128, 16, "uniform:4096", 256), {"shared_prefix": 0.5}),
        ("samples B4 L4096 50% shared", (4, 32, 8, 128, 16, "uniform:4096", 256), {"shared_prefix": 0.5}),
        ("fp8 samples B16 L4096 50% shared", (16, 32, 8, 128, 16, "uniform:4096", 256),
         {"shared_prefix": 0.5, "fmt": "fp8"}),
        ("bf16 samples B8 L8192 50% shared", (8, 32, 8, 128, 16, "uniform:8192", 256),
         {"shared_prefix": 0.5, "fmt": "bf16"}),
    ]
    for runs in (True, False)
]

SWEEPS = {"coarse": COARSE, "reserved": RESERVED, "small": SMALL, "mid": MID, "xcd": XCD, "rows": ROWS,
          "prefix": PREFIX}


def shapes(names):
    """Shapes of the named sweeps ("all": every sweep), without repeats."""
    names = list(SWEEPS) if names == ["all"] else names
    out, seen = [], set()
    for name in names:
        if name not in SWEEPS:
            raise ValueError(f"unknown sweep {name!r}; choose from {sorted(SWEEPS)} or all")
        for shape in SWEEPS[name]:
            if shape not in seen:
                seen.add(shape)
                out.append((name, shape))
    return out


def metadata(shape, seed=7):
    """Layout, page table and lengths of a shape (host arrays)."""
    kind, _, value = shape.lengths.partition(":")
    rng = np.random.default_rng(seed)
    if kind == "workload":
        # The named workload's own page table and lengths (shared pages
        # included), widened with padding columns for a reserve.
        w = make_workload(value)
        longest = max(1, int(w.lengths.max()))
        width = max(w.table.shape[1], math.ceil(longest * shape.reserve / shape.page_size))
        table = np.full((shape.batch, width), -1, dtype=np.int32)
        table[:, :w.table.shape[1]] = w.table
        return w.layout, table, w.lengths.astype(np.int32), longest * shape.reserve
    context = int(value)
    if kind == "reference":
        _, _, lengths = make_metadata(shape.batch, shape.query_heads, shape.kv_heads, shape.head_dim, context,
                                      shape.page_size, seed=123)
    elif kind == "ragged":
        lengths = rng.integers(0, context + 1, size=shape.batch, dtype=np.int32)
        lengths[0] = context
        if shape.batch > 2:
            lengths[rng.integers(1, shape.batch)] = 0
    elif kind == "skewed":
        lengths = rng.integers(0, context // 2 + 1, size=shape.batch, dtype=np.int32)
        lengths[0] = context
    elif kind == "uniform":
        lengths = np.full(shape.batch, context, dtype=np.int32)
    else:
        raise ValueError(f"unknown lengths {shape.lengths!r}")
    longest = max(1, int(lengths.max()))
    width = math.ceil(longest * shape.reserve / shape.page_size)
    shared = int(math.ceil(longest / shape.page_size) * shape.shared_prefix)  # of the context, not the reserve
    private = rng.permutation(shape.batch * (width - shared)).reshape(shape.batch, width - shared)
    table = np.empty((shape.batch, width), dtype=np.int32)
    table[:, :shared] = np.arange(shared, dtype=np.int32)[None, :]
    table[:, shared:] = private + shared
    for row, length in enumerate(lengths):
        table[row, math.ceil(int(length) / shape.page_size):] = -1
    layout = Layout(shape.batch, shape.query_heads, shape.kv_heads, shape.head_dim, shape.page_size,
                    shared + shape.batch * (width - shared))
    return layout, table, lengths.astype(np.int32), longest * shape.reserve


def _tensors(torch, layout, fmt, device, seed):
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    cache = (layout.physical_pages, layout.page_size, layout.kv_heads, layout.head_dim)
    q_dtype = {"f16": torch.float16, "fp8": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[fmt]
    q = torch.randn((layout.batch, layout.query_heads, layout.head_dim), generator=g, device=device).to(q_dtype)
    k = torch.randn(cache, generator=g, device=device)
    v = torch.randn(cache, generator=g, device=device)
    if fmt == "fp8":
        largest = float(torch.finfo(torch.float8_e4m3fn).max)
        scale = 6.0 / largest  # codes of |x| / scale, clamped into range (e4m3fn has no infinity)
        k, v = ((x / scale).clamp(-largest, largest).to(torch.float8_e4m3fn) for x in (k, v))
        return q, k, v, scale, scale
    return q, k.to(q_dtype), v.to(q_dtype), 1.0, 1.0


def _graph_us(torch, fn, steps, warm=2):
    """Device us per call of `steps` calls captured back to back in one graph."""
    for i in range(warm):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for i in range(steps):
                fn(i)
    torch.cuda.current_stream().wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    best = math.inf
    for _ in range(2):
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        best = min(best, start.elapsed_time(end))
    del graph
    return best * 1e3 / steps


def run(names, steps=200, merge="serial", out=sys.stdout, log=None):
    """Times every shape of the named sweeps; prints one JSON line per shape."""
    import torch

    from .runtime import DecodePlan

    device = torch.device("cuda", 0)
    records = []
    for sweep, shape in shapes(names):
        layout, table, lengths, max_context = metadata(shape)
        q, k0, v0, k_scale, v_scale = _tensors(torch, layout, shape.fmt, device, seed=11)
        set_bytes = 2 * k0.numel() * k0.element_size()
        sets = max(1, math.ceil(ROTATION_BYTES / set_bytes))
        ks = [k0] + [k0.clone() for _ in range(sets - 1)]
        vs = [v0] + [v0.clone() for _ in range(sets - 1)]
        plan = DecodePlan(layout, table, lengths, device=device, split_tokens=shape.split_tokens, merge=merge,
                          max_context=int(min(max_context, table.shape[1] * layout.page_size)))
        if not shape.runs:
            plan._prefix_runs = None
        scales = {"k_scale": k_scale, "v_scale": v_scale}
        ext = plan._extension
        if shape.bounds:
            def call(i):
                plan.run(q, ks[i % sets], vs[i % sets], **scales)
        else:
            def call(i):
                ext.decode(q, ks[i % sets], vs[i % sets], plan._table, plan._lengths, plan._numerator, plan._stats,
                           plan._out, shape.split_tokens, plan._merge_mode, k_scale, v_scale, plan._unshared_pages,
                           plan._ragged_lengths, None)
        record = {"sweep": sweep, "shape": shape.name, "lengths": shape.lengths, "fmt": shape.fmt,
                  "split_tokens": shape.split_tokens, "reserve": shape.reserve, "bounds": shape.bounds,
                  "runs": shape.runs,
                  "kv_bytes_per_call": int(lengths.astype(np.int64).sum()) * layout.kv_heads * layout.head_dim * 2
                  * k0.element_size(), "kv_buffer_sets": sets}
        record["us_per_call"] = round(_graph_us(torch, call, steps), 3)
        if shape.bounds:
            record["plan"] = plan.launch_plan(q.dtype, k0.dtype)
            record["partition_us"] = round(_graph_us(torch, lambda i: plan.run_partial(q, ks[i % sets], vs[i % sets],
                                                                                      **scales), steps), 3)
        staged = {}
        for c in shape.coarse:
            splits = math.ceil(plan.splits / c)
            num, stats = plan._stage_workspace(splits)
            bounds = plan._length_bounds()

            def stage(i, c=c, num=num, stats=stats, bounds=bounds):
                ext.partial(q, ks[i % sets], vs[i % sets], plan._table, plan._lengths, num, stats,
                            c * shape.split_tokens, k_scale, v_scale, plan._unshared_pages, plan._ragged_lengths,
                            bounds, plan._prefix_runs)
                ext.merge(num, stats, plan._out, plan._lengths, layout.page_size, table.shape[1],
                          c * shape.split_tokens, plan._merge_mode)
            staged[f"x{c}"] = round(_graph_us(torch, stage, steps), 3)
        if staged:
            record["staged_us_by_kernel_split"] = staged
        out.write(json.dumps(record) + "\n")
        out.flush()
        if log is not None:
            log(f"{shape.name}: {record['us_per_call']} us/call" + (f", staged {staged}" if staged else ""))
        records.append(record)
        del ks, vs, plan, q, k0, v0
        torch.cuda.empty_cache()
    return records
