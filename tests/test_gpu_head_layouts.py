"""Head layouts that reach the less common paths of the partition kernels.

GQA groups that do not fill a head tile (3, 5, 12, 24), groups split into
several head tiles (24, 32: two tiles of 16 in the matrix-core kernel, three
or four of 8 in the FP32 kernel), KV head counts that give workgroups of an
odd number of heads (3, 5, 6, 7, 12; 7 stays one workgroup of 7 waves) or
several head groups per token row (12, 16, 20, and 11, whose prime count
gives one head per workgroup: the streaming-load variants), each against
the FP64 oracle on ragged lengths with empty rows.
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, host, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import host_tensors  # noqa: E402

pytestmark = pytest.mark.gpu

HEADS = [(12, 4), (24, 1), (64, 2), (40, 8), (36, 12), (10, 5), (96, 3), (48, 16), (18, 6), (14, 7), (22, 11),
         (40, 20)]


def problem(query_heads, kv_heads, dim, seed):
    batch, page, width = 3, 16, 12
    layout = Layout(batch, query_heads, kv_heads, dim, page, batch * width)
    rng = np.random.default_rng(seed)
    table = rng.permutation(batch * width).reshape(batch, width).astype(np.int32)
    lengths = np.array([width * page, 0, 77], dtype=np.int32)
    table[1, :] = -1
    table[2, 5:] = -1
    return layout, table, lengths


@pytest.mark.parametrize("query_heads,kv_heads", HEADS)
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("dim", [64, 128])
def test_head_layouts(query_heads, kv_heads, dtype, dim):
    announce(f"heads {query_heads}/{kv_heads} dim={dim} {dtype}")
    layout, table, lengths = problem(query_heads, kv_heads, dim, seed=query_heads * 7 + kv_heads)
    q, k, v = (torch.from_numpy(x).to(dtype).cuda() for x in host_tensors(layout, dtype=np.float32, seed=3))
    expected = dense_attention(*host(q, k, v), table, lengths)
    for merge in ("serial", "shared"):
        plan = DecodePlan(layout, table, lengths, split_tokens=64, merge=merge)
        actual = plan.run(q, k, v).cpu().numpy()
        assert_parity(actual, expected, dtype)
        np.testing.assert_array_equal(actual[1], 0.0)


@pytest.mark.parametrize("query_heads,kv_heads", [(24, 1), (36, 12), (96, 3)])
@pytest.mark.parametrize("kv_dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_head_layouts_other_formats(query_heads, kv_heads, kv_dtype):
    announce(f"heads {query_heads}/{kv_heads} {kv_dtype}")
    layout, table, lengths = problem(query_heads, kv_heads, 128, seed=5)
    qf, kf, vf = host_tensors(layout, dtype=np.float32, seed=4)
    q = torch.from_numpy(qf).to(torch.bfloat16)
    if kv_dtype == torch.bfloat16:
        k, v, k_scale, v_scale = torch.from_numpy(kf).to(kv_dtype), torch.from_numpy(vf).to(kv_dtype), 1.0, 1.0
        exact = (q.double().numpy(), k.double().numpy(), v.double().numpy())
    else:
        largest = float(torch.finfo(kv_dtype).max)
        k_scale, v_scale = float(np.abs(kf).max()) / largest, float(np.abs(vf).max()) / largest
        k = (torch.from_numpy(kf) / k_scale).to(kv_dtype)
        v = (torch.from_numpy(vf) / v_scale).to(kv_dtype)
        exact = (q.double().numpy(), k.double().numpy() * k_scale, v.double().numpy() * v_scale)
    plan = DecodePlan(layout, table, lengths, split_tokens=64)
    actual = plan.run(q.cuda(), k.cuda(), v.cuda(), k_scale=k_scale, v_scale=v_scale).cpu().numpy()
    assert_parity(actual, dense_attention(*exact, table, lengths), torch.bfloat16)
