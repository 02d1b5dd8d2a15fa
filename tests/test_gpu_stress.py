"""1,000 randomized cases, restating the reference's stress recipe.

Recipe of reference results/2026-10-31-h100/diagnostic/stress-clean.py:6-19
(restated, not run): generator default_rng(97531); per case batch in {1,2,3},
kv heads in {1,2,4}, heads = kv * {1,2,4,8}, dim in {64,128}, page in
{16,32}, context from a fixed list; seed % 3 empties the last row, seed % 5
maps every page to page 0, odd seeds use FP16, seed % 7 scales q and k by 20;
split drawn from {1,7,31,128,256,511}; both merges. Each case is gated at the
parity bar of tests/gpu_util.py (unscaled cases) or at the reference's 3e-3
(x20-scaled cases, whose logits reach ~1e3).
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, host, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import make_metadata, make_tensors  # noqa: E402

pytestmark = pytest.mark.gpu

CASES = 1000


def test_thousand_randomized_cases():
    rng = np.random.default_rng(97531)
    worst = 0.0
    for seed in range(CASES):
        b = int(rng.choice([1, 2, 3]))
        kv = int(rng.choice([1, 2, 4]))
        h = kv * int(rng.choice([1, 2, 4, 8]))
        d = int(rng.choice([64, 128]))
        page = int(rng.choice([16, 32]))
        length = int(rng.choice([1, 15, 16, 17, 31, 32, 33, 127, 129, 257, 513]))
        layout, table, lengths = make_metadata(b, h, kv, d, length, page, seed=seed)
        if seed % 3 == 0:
            lengths[-1] = 0
            table[-1, :] = -1
        if seed % 5 == 0:
            table[table >= 0] = 0
        dtype = torch.float16 if seed % 2 else torch.float32
        q, k, v = make_tensors(layout, dtype=dtype, seed=seed + 10000)
        scaled = seed % 7 == 0
        if scaled:
            q.mul_(20)
            k.mul_(20)
        ref = dense_attention(*host(q, k, v), table, lengths)
        for merge in ("serial", "shared"):
            split = int(rng.choice([1, 7, 31, 128, 256, 511]))
            if seed % 100 == 0 and merge == "serial":
                announce(f"stress case {seed} worst so far {worst:.3e}")
            plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
            out = plan.run(q, k, v).cpu().numpy()
            worst = max(worst, float(np.max(np.abs(out - ref))))
            try:
                if scaled:
                    np.testing.assert_allclose(out, ref, atol=3e-3, rtol=3e-3)
                else:
                    assert_parity(out, ref, dtype)
            except AssertionError as exc:
                raise AssertionError(f"case {seed} merge={merge} split={split} {layout} "
                                     f"lengths={lengths.tolist()} dtype={dtype}") from exc
    announce(f"stress: {CASES} cases x 2 merges, max abs error {worst:.3e}")


COMBINE_CASES = 300


def test_randomized_combined_quarter_cases():
    """Randomized few-KV-head shapes (the quarter-combining workgroup layouts).

    One or two KV heads with groups of 16, 24, 32 or 48 query heads (16-head
    tiles: four quarters per workgroup for one tile, two for up to two tiles
    per KV head pair), FP16 / BF16 / FP8-e4m3 K/V, ragged and empty rows,
    small splits (rows of up to a few hundred states) and both merges, each
    against the FP64 oracle on the values the device holds. Most of these
    grids are smaller than the device and keep four states per partition; the
    larger ones combine (see the large-grid test below).
    """
    rng = np.random.default_rng(24680)
    worst = 0.0
    for seed in range(COMBINE_CASES):
        b = int(rng.choice([1, 2, 3, 5]))
        kv = int(rng.choice([1, 2]))
        h = kv * int(rng.choice([16, 24, 32, 48]))
        d = int(rng.choice([64, 128]))
        page = int(rng.choice([16, 32]))
        length = int(rng.choice([1, 17, 64, 129, 300, 513, 1000]))
        layout, table, lengths = make_metadata(b, h, kv, d, length, page, seed=seed)
        if seed % 4 == 0:
            lengths[-1] = 0
            table[-1, :] = -1
        fmt = ("f16", "bf16", "e4m3")[seed % 3]
        qf, kf, vf = (t.float() for t in make_tensors(layout, dtype=torch.float32, seed=seed + 20000))
        if fmt == "f16":
            q, k, v = qf.half(), kf.half(), vf.half()
            k_scale = v_scale = 1.0
            exact = host(q.double(), k.double(), v.double())
        elif fmt == "bf16":
            q, k, v = qf.bfloat16(), kf.bfloat16(), vf.bfloat16()
            k_scale = v_scale = 1.0
            exact = host(q.double(), k.double(), v.double())
        else:
            largest = float(torch.finfo(torch.float8_e4m3fn).max)
            k_scale, v_scale = float(kf.abs().max()) / largest, float(vf.abs().max()) / largest
            q = qf.half()
            k = (kf / k_scale).to(torch.float8_e4m3fn)
            v = (vf / v_scale).to(torch.float8_e4m3fn)
            exact = (host(q.double())[0], host(k.double())[0] * k_scale, host(v.double())[0] * v_scale)
        ref = dense_attention(*exact, table, lengths)
        for merge in ("serial", "shared"):
            split = int(rng.choice([16, 48, 64, 128, 256]))
            if seed % 50 == 0 and merge == "serial":
                announce(f"combine stress case {seed} worst so far {worst:.3e}")
            plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
            out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).cpu().numpy()
            worst = max(worst, float(np.max(np.abs(out - ref))))
            try:
                assert_parity(out, ref, torch.float16)
            except AssertionError as exc:
                raise AssertionError(f"case {seed} merge={merge} split={split} {layout} {fmt} "
                                     f"lengths={lengths.tolist()}") from exc
    announce(f"combine stress: {COMBINE_CASES} cases x 2 merges, max abs error {worst:.3e}")


LARGE_GRID_CASES = 30


def test_randomized_combined_quarters_large_grids():
    """Randomized few-KV-head shapes with grids that fill the device, so the
    partition kernel combines its quarters (splits of 64 or 128 tokens: every
    quarter holds tokens), FP16 / BF16 / FP8-e4m3 K/V, ragged and empty rows,
    both merges, against the FP64 oracle."""
    rng = np.random.default_rng(13579)
    worst = 0.0
    for seed in range(LARGE_GRID_CASES):
        b = int(rng.choice([24, 32]))
        kv = int(rng.choice([1, 2]))
        h = kv * int(rng.choice([16, 24]))
        d = int(rng.choice([64, 128]))
        length = int(rng.choice([1100, 1600]))
        layout, table, lengths = make_metadata(b, h, kv, d, length, 16, seed=seed)
        lengths[1] = 0
        table[1, :] = -1
        fmt = ("f16", "bf16", "e4m3")[seed % 3]
        qf, kf, vf = make_tensors(layout, dtype=torch.float32, seed=seed + 30000)
        if fmt == "e4m3":
            largest = float(torch.finfo(torch.float8_e4m3fn).max)
            k_scale, v_scale = float(kf.abs().max()) / largest, float(vf.abs().max()) / largest
            q, k, v = qf.half(), (kf / k_scale).to(torch.float8_e4m3fn), (vf / v_scale).to(torch.float8_e4m3fn)
            exact = (host(q.double())[0], host(k.double())[0] * k_scale, host(v.double())[0] * v_scale)
        else:
            dt = torch.float16 if fmt == "f16" else torch.bfloat16
            q, k, v = qf.to(dt), kf.to(dt), vf.to(dt)
            k_scale = v_scale = 1.0
            exact = host(q.double(), k.double(), v.double())
        ref = dense_attention(*exact, table, lengths)
        for merge in ("serial", "shared"):
            split = int(rng.choice([64, 128]))
            plan = DecodePlan(layout, table, lengths, split_tokens=split, merge=merge)
            out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).cpu().numpy()
            worst = max(worst, float(np.max(np.abs(out - ref))))
            try:
                assert_parity(out, ref, torch.float16)
            except AssertionError as exc:
                raise AssertionError(f"case {seed} merge={merge} split={split} {layout} {fmt}") from exc
        if seed % 10 == 0:
            announce(f"large-grid combine case {seed} worst so far {worst:.3e}")
    announce(f"large-grid combine stress: {LARGE_GRID_CASES} cases x 2 merges, max abs error {worst:.3e}")
