"""Deterministic paged-decode workloads.

``make_metadata`` restates reference ``src/paged_decode/workload.py:7-22`` draw
for draw (same NumPy generator calls in the same order), so a seed yields the
same page table and lengths as the reference. ``make_tensors`` keeps the
reference signature (``workload.py:25-35``) but draws values with NumPy on the
host and copies them to the device, so the same seed gives the same values on
every device; the reference draws with a device-dependent torch generator.

``make_workload`` builds the named decode shapes this operator is measured and
tested on: Llama-3-8B geometry (FP16, BF16, FP8 K/V), ragged/shared-prefix
stress, large-batch MQA, long-context MHA, the small FP32 case, and the
reference's own benchmark shape at batch 1, 4 and 16.
"""
from dataclasses import dataclass, field
import math

import numpy as np

from .layout import Layout


def make_metadata(batch, heads, kv_heads, dim, context, page_size, *, seed=123, ragged=True):
    """Shuffled one-owner page table, ragged lengths and ``-1`` padding.

    Lengths are drawn from ``[max(1, context // 4), context]`` and the first
    sequence always has ``context`` tokens.
    """
    if min(batch, heads, kv_heads, dim, context, page_size) <= 0:
        raise ValueError("workload dimensions must be positive")
    rng = np.random.default_rng(seed)
    width = math.ceil(context / page_size)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = rng.integers(max(1, context // 4), context + 1, size=batch, dtype=np.int32)
    if not ragged:
        lengths.fill(context)
    lengths[0] = context
    layout = Layout(batch, heads, kv_heads, dim, page_size, batch * width)
    for row, length in enumerate(lengths):
        table[row, math.ceil(int(length) / page_size):] = -1
    return layout, table, lengths


def host_tensors(layout, *, dtype=np.float16, seed=123):
    """Seeded N(0,1) ``q [B,Hq,D]`` and ``k, v [P,T,Hkv,D]`` as NumPy arrays."""
    rng = np.random.default_rng(seed)
    cache_shape = (layout.physical_pages, layout.page_size, layout.kv_heads, layout.head_dim)
    q = rng.standard_normal((layout.batch, layout.query_heads, layout.head_dim), dtype=np.float32)
    k = rng.standard_normal(cache_shape, dtype=np.float32)
    v = rng.standard_normal(cache_shape, dtype=np.float32)
    return q.astype(dtype), k.astype(dtype), v.astype(dtype)


def make_tensors(layout, *, device="cuda", dtype=None, seed=123):
    """Seeded ``(q, k, v)`` torch tensors on ``device`` (float16 by default)."""
    import torch

    dtype = torch.float16 if dtype is None else dtype
    np_dtype = {torch.float16: np.float16, torch.float32: np.float32}.get(dtype)
    if np_dtype is None:
        # Other dtypes are produced through float32 so callers can still build
        # rejected inputs (e.g. float64) for negative tests.
        q, k, v = host_tensors(layout, dtype=np.float32, seed=seed)
        return tuple(torch.from_numpy(x).to(device=device, dtype=dtype) for x in (q, k, v))
    q, k, v = host_tensors(layout, dtype=np_dtype, seed=seed)
    return tuple(torch.from_numpy(x).to(device) for x in (q, k, v))


@dataclass
class Workload:
    """A named decode problem: metadata, split size, dtype and value seed."""

    name: str
    layout: Layout
    table: np.ndarray
    lengths: np.ndarray
    split_tokens: int
    dtype: type
    seed: int
    description: str
    heavy_key_fraction: float = 0.0
    split_sweep: tuple = field(default_factory=tuple)
    q_format: str = ""   # "bf16" for a bfloat16 q (and K/V unless kv_format says otherwise)
    kv_format: str = ""  # "e4m3" / "e5m2": FP8 K/V with per-tensor scales

    def _values(self):
        q, k, v = host_tensors(self.layout, dtype=np.float32, seed=self.seed)
        if self.heavy_key_fraction:
            # A seeded 5% of key entries scaled x20 stresses max correction.
            mask_rng = np.random.default_rng(self.seed + 1)
            k[mask_rng.random(k.shape) < self.heavy_key_fraction] *= 20.0
        return q, k, v

    @property
    def native(self):
        """True when q/k/v are NumPy-representable (float16 or float32)."""
        return not self.q_format and not self.kv_format

    def host_tensors(self):
        """``q, k, v`` as NumPy arrays holding exactly the values the device uses.

        float16/float32 workloads return arrays in that dtype. BF16 workloads
        return float32 arrays of the bfloat16 values; FP8 workloads return
        float64 arrays of ``code * scale`` (exact), the values the attention
        runs over.
        """
        if self.native:
            q, k, v = self._values()
            return q.astype(self.dtype), k.astype(self.dtype), v.astype(self.dtype)
        q, k, v, k_scale, v_scale = self.tensors("cpu")
        if self.kv_format:
            return (q.float().numpy(), k.double().numpy() * k_scale, v.double().numpy() * v_scale)
        return q.float().numpy(), k.float().numpy(), v.float().numpy()

    def tensors(self, device):
        """``(q, k, v, k_scale, v_scale)``: torch tensors in the storage formats on ``device``."""
        import torch

        q, k, v = self._values()
        q_dtype = torch.bfloat16 if self.q_format == "bf16" else torch.from_numpy(np.zeros(0, self.dtype)).dtype
        qt = torch.from_numpy(q).to(q_dtype)
        if self.kv_format:
            fp8 = torch.float8_e4m3fn if self.kv_format == "e4m3" else torch.float8_e5m2
            largest = float(torch.finfo(fp8).max)
            k_scale = float(np.abs(k).max()) / largest
            v_scale = float(np.abs(v).max()) / largest
            kt = (torch.from_numpy(k) / k_scale).to(fp8)
            vt = (torch.from_numpy(v) / v_scale).to(fp8)
        else:
            k_scale = v_scale = 1.0
            kt, vt = torch.from_numpy(k).to(q_dtype), torch.from_numpy(v).to(q_dtype)
        return qt.to(device), kt.to(device), vt.to(device), k_scale, v_scale

    @property
    def element_size(self):
        """Bytes per stored K/V element."""
        if self.kv_format:
            return 1
        if self.q_format == "bf16":
            return 2
        return np.dtype(self.dtype).itemsize

    @property
    def format_label(self):
        if self.kv_format:
            return f"fp8-{self.kv_format} K/V, {'bf16' if self.q_format == 'bf16' else 'f16'} q"
        if self.q_format == "bf16":
            return "bf16"
        return "f16" if self.dtype == np.float16 else "f32"


def _shuffled_table(rng, batch, width):
    return rng.permutation(batch * width).reshape(batch, width).astype(np.int32)


def _pad(table, lengths, page_size):
    for row, length in enumerate(lengths):
        table[row, (int(length) + page_size - 1) // page_size:] = -1
    return table


def make_workload(name, *, seed=None, split_tokens=None):
    """Build one of the named workloads (see ``WORKLOAD_NAMES``)."""
    if name == "fp32_b2_ragged":
        seed = 0 if seed is None else seed
        rng = np.random.default_rng(seed)
        batch, width, page = 2, 16, 16
        lengths = np.array([100, 256], dtype=np.int32)
        table = _pad(_shuffled_table(rng, batch, width), lengths, page)
        layout = Layout(batch, 8, 2, 64, page, batch * width)
        return Workload(name, layout, table, lengths, split_tokens or 256, np.float32, seed,
                        "FP32 B2 Hq8 Hkv2 D64 T16, lengths [100,256], shuffled pages")
    if name == "llama3_8b_b4_l4096":
        seed = 2 if seed is None else seed
        rng = np.random.default_rng(seed)
        batch, page, context = 4, 16, 4096
        width = context // page
        lengths = np.full(batch, context, dtype=np.int32)
        table = _shuffled_table(rng, batch, width)
        layout = Layout(batch, 32, 8, 128, page, batch * width)
        return Workload(name, layout, table, lengths, split_tokens or 256, np.float16, seed,
                        "Llama-3-8B decode: FP16 B4 Hq32 Hkv8 D128 T16, uniform 4096, shuffled pages")
    if name == "ragged_shared_b16":
        seed = 3 if seed is None else seed
        rng = np.random.default_rng(seed)
        batch, page, context = 16, 32, 8192
        width = context // page
        shared = width // 4  # a 25% shared prefix of physical pages
        lengths = rng.integers(0, context + 1, size=batch, dtype=np.int32)
        lengths[rng.integers(0, batch)] = 0  # at least one empty context
        private = rng.permutation(batch * (width - shared)).reshape(batch, width - shared)
        table = np.empty((batch, width), dtype=np.int32)
        table[:, :shared] = np.arange(shared, dtype=np.int32)[None, :]
        table[:, shared:] = private + shared
        table = _pad(table, lengths, page)
        layout = Layout(batch, 32, 8, 128, page, shared + batch * (width - shared))
        return Workload(name, layout, table, lengths, split_tokens or 128, np.float16, seed,
                        "FP16 B16 Hq32 Hkv8 D128 T32, lengths U[0,8192] incl. 0, 25% shared prefix pages")
    if name == "mqa_b128_l1024":
        seed = 4 if seed is None else seed
        rng = np.random.default_rng(seed)
        batch, page, context = 128, 16, 1024
        width = context // page
        lengths = np.full(batch, context, dtype=np.int32)
        table = _shuffled_table(rng, batch, width)
        layout = Layout(batch, 16, 1, 64, page, batch * width)
        return Workload(name, layout, table, lengths, split_tokens or 256, np.float16, seed,
                        "MQA FP16 B128 Hq16 Hkv1 D64 T16, uniform 1024, 5% of keys x20",
                        heavy_key_fraction=0.05)
    if name == "long_mha_b1_l32768":
        seed = 5 if seed is None else seed
        rng = np.random.default_rng(seed)
        batch, page, context = 1, 16, 32768
        width = context // page
        lengths = np.full(batch, context, dtype=np.int32)
        table = _shuffled_table(rng, batch, width)
        layout = Layout(batch, 32, 32, 128, page, batch * width)
        return Workload(name, layout, table, lengths, split_tokens or 512, np.float16, seed,
                        "Long-context MHA FP16 B1 Hq32 Hkv32 D128 T16, context 32768",
                        split_sweep=(128, 256, 512, 1024))
    if name in ("llama3_8b_b4_l4096_bf16", "llama3_8b_b4_l4096_fp8"):
        base = make_workload("llama3_8b_b4_l4096", seed=seed, split_tokens=split_tokens)
        base.name = name
        if name.endswith("bf16"):
            base.q_format = "bf16"
            base.description = base.description.replace("FP16", "BF16")
        else:
            base.kv_format = "e4m3"
            base.description = base.description.replace("FP16", "FP16 q, FP8 e4m3 K/V with per-tensor scales,")
        return base
    if name in _REFERENCE_BENCH:
        # The reference's own benchmark shape (benchmarks/bench_competitive.py
        # defaults: 32/8 heads, D128, context 4096, page 16, split 256, seed
        # 123) at the batches its published results cover
        # (results/2026-10-31-h100/SUMMARY.md:34-40): make_metadata's ragged
        # lengths, e.g. [4096, 2311, 2289, 2568] at batch 4.
        batch = _REFERENCE_BENCH[name]
        layout, table, lengths = make_metadata(batch, 32, 8, 128, 4096, 16, seed=123)
        return Workload(name, layout, table, lengths, split_tokens or 256, np.float16, 123 if seed is None else seed,
                        f"Reference benchmark shape: FP16 B{batch} Hq32 Hkv8 D128 T16, make_metadata(seed=123) "
                        "ragged lengths up to 4096")
    raise ValueError(f"unknown workload {name!r}; choose from {WORKLOAD_NAMES}")


_REFERENCE_BENCH = {"reference_b1_l4096": 1, "reference_b4_l4096": 4, "reference_b16_l4096": 16}

WORKLOAD_NAMES = ("fp32_b2_ragged", "llama3_8b_b4_l4096", "ragged_shared_b16",
                  "mqa_b128_l1024", "long_mha_b1_l32768", "llama3_8b_b4_l4096_bf16", "llama3_8b_b4_l4096_fp8",
                  *_REFERENCE_BENCH)
