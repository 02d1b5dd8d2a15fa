"""BF16 inputs and FP8 (OCP e4m3 / e5m2) K/V against the FP64 oracle.

The oracle runs on exactly the values the device uses: the bfloat16 inputs
widened, and FP8 codes times their per-tensor scale (in float64, exact). The
bar is the FP16 one (2e-3 absolute, and the reference's 5e-4 gate); the only
extra rounding on the device is the split of the softmax weights into high and
low 16-bit parts for the P.V matrix product.
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import host_tensors  # noqa: E402

pytestmark = pytest.mark.gpu

FORMATS = [
    (torch.bfloat16, None),
    (torch.float16, torch.float8_e4m3fn),
    (torch.float16, torch.float8_e5m2),
    (torch.bfloat16, torch.float8_e4m3fn),
    (torch.bfloat16, torch.float8_e5m2),
]


def quantized(layout, q_dtype, kv_dtype, seed, key_boost=1.0):
    """Device tensors in the formats, scales, and the exact float64 values they hold."""
    q, k, v = host_tensors(layout, dtype=np.float32, seed=seed)
    k = k * key_boost
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


@pytest.mark.parametrize("q_dtype,kv_dtype", FORMATS)
@pytest.mark.parametrize("dim,page_size", [(64, 16), (128, 32)])
@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_formats_ragged(q_dtype, kv_dtype, dim, page_size, merge):
    announce(f"formats q={q_dtype} kv={kv_dtype} dim={dim} page={page_size} merge={merge}")
    layout = Layout(4, 8, 2, dim, page_size, 32)
    table = np.random.default_rng(5).permutation(32).reshape(4, 8).astype(np.int32)
    lengths = np.array([0, 1, page_size + 1, 127], dtype=np.int32)
    for b, length in enumerate(lengths):
        table[b, (int(length) + page_size - 1) // page_size:] = -1
    (q, k, v), (k_scale, v_scale), exact = quantized(layout, q_dtype, kv_dtype, seed=dim + page_size)
    plan = DecodePlan(layout, table, lengths, split_tokens=33, merge=merge)
    out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).cpu().numpy()
    assert_parity(out, dense_attention(*exact, table, lengths), torch.float16)
    np.testing.assert_array_equal(out[0], 0.0)


@pytest.mark.parametrize("q_dtype,kv_dtype", FORMATS)
def test_formats_group_of_sixteen_with_heavy_keys(q_dtype, kv_dtype):
    """MQA-style group of 16 query heads (one 16-head tile), keys x20 for max correction."""
    announce(f"formats mqa q={q_dtype} kv={kv_dtype}")
    layout = Layout(3, 16, 1, 64, 16, 3 * 40)
    table = np.arange(3 * 40, dtype=np.int32).reshape(3, 40)
    lengths = np.array([640, 17, 333], dtype=np.int32)
    (q, k, v), (k_scale, v_scale), exact = quantized(layout, q_dtype, kv_dtype, seed=9, key_boost=3.0)
    plan = DecodePlan(layout, table, lengths, split_tokens=128)
    out = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).cpu().numpy()
    assert_parity(out, dense_attention(*exact, table, lengths), torch.float16)


def test_scales_equal_dequantized_inputs():
    """FP16 cache with scales == the same cache pre-multiplied (scales fold exactly)."""
    announce("scales fold")
    layout = Layout(2, 8, 2, 128, 16, 16)
    table = np.arange(16, dtype=np.int32).reshape(2, 8)
    lengths = np.array([128, 70], dtype=np.int32)
    q, k, v = (torch.from_numpy(x).cuda() for x in host_tensors(layout, dtype=np.float16, seed=4))
    plan = DecodePlan(layout, table, lengths)
    scaled = plan.run(q, k, v, k_scale=0.5, v_scale=0.25).clone()
    direct = plan.run(q, k * 0.5, v * 0.25)
    torch.testing.assert_close(scaled, direct, rtol=1e-6, atol=1e-6)


def test_rejects_invalid_formats_and_scales():
    layout = Layout(1, 8, 2, 64, 16, 8)
    plan = DecodePlan(layout, np.arange(8, dtype=np.int32)[None], np.array([127]))
    q, k, v = (torch.from_numpy(x).cuda() for x in host_tensors(layout, dtype=np.float32, seed=1))
    with pytest.raises(TypeError):
        plan.run(q, k.to(torch.float8_e4m3fn), v.to(torch.float8_e4m3fn))   # FP8 K/V need a 16-bit q
    with pytest.raises(TypeError):
        plan.run(q.half(), k.bfloat16(), v.bfloat16())                         # mixed 16-bit formats
    with pytest.raises(TypeError):
        plan.run(q.half(), k.to(torch.float8_e4m3fn), v.to(torch.float8_e5m2))
    for bad in (0.0, -1.0, float("nan"), float("inf"), True):
        with pytest.raises(ValueError):
            plan.run(q.half(), k.half(), v.half(), k_scale=bad)
