"""The Python snippets of INTEGRATION.md run as written, on the GPU.

The quick start (section 2), the captured decode loop (section 2.1) and the
ctypes call (section 4) are taken from the document itself, so document and
test cannot drift, and run in a namespace that supplies the names each
snippet leaves to the reader (sizes, device buffers, a fill function). Each
result is compared with the FP64 oracle. The reference-side rebinding
(section 3) is exercised by tests/test_gpu_reference_call.py.
"""
import math
import re
from pathlib import Path

import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle import fp64  # noqa: E402
from paged_decode.workload import host_tensors, make_metadata  # noqa: E402

pytestmark = pytest.mark.gpu

INTEGRATION = Path(__file__).resolve().parent.parent / "INTEGRATION.md"


def python_blocks():
    return re.findall(r"```python\n(.*?)```", INTEGRATION.read_text(), flags=re.S)


def block(needle):
    found = [b for b in python_blocks() if needle in b]
    assert len(found) == 1, needle
    return found[0]


def test_quick_start_snippet():
    announce("INTEGRATION quick start")
    namespace = {}
    exec(compile(block("make_metadata(4, 32, 8, 128, 4096, 16, seed=123)"), str(INTEGRATION), "exec"), namespace)
    torch.cuda.synchronize()
    layout, table, lengths = namespace["layout"], namespace["table"], namespace["lengths"]
    q, k, v = (namespace[n].double().cpu().numpy() for n in ("q", "k", "v"))
    assert_parity(namespace["out"].cpu().numpy(), fp64.dense_attention(q, k, v, table, lengths), torch.float16)


def test_captured_decode_loop_snippet():
    announce("INTEGRATION captured decode loop")
    layout, table, lengths = make_metadata(2, 8, 2, 64, 4096, 16, seed=7)  # tables wide enough for max_context=4096
    lengths = (lengths // 2).astype(np.int32)  # room to append
    q, k, v = (torch.from_numpy(x).half().cuda() for x in host_tensors(layout, dtype=np.float32, seed=8))
    q_step = q.clone()
    k_step = torch.empty((layout.batch, layout.kv_heads, layout.head_dim), device="cuda", dtype=torch.float16)
    v_step = torch.empty_like(k_step)
    rng = np.random.default_rng(9)
    host = {"k": k.double().cpu().numpy(), "v": v.double().cpu().numpy(), "lengths": lengths.copy()}

    def fill(qs, ks, vs):
        new_k = rng.standard_normal(ks.shape).astype(np.float16)
        new_v = rng.standard_normal(vs.shape).astype(np.float16)
        qs.copy_(torch.from_numpy(rng.standard_normal(qs.shape).astype(np.float16)))
        ks.copy_(torch.from_numpy(new_k))
        vs.copy_(torch.from_numpy(new_v))
        host["q"] = qs.double().cpu().numpy()
        host["k"], _ = fp64.append_advance(host["k"], table, host["lengths"], new_k[:, None].astype(np.float64),
                                          max_context=4096)
        host["v"], host["lengths"] = fp64.append_advance(host["v"], table, host["lengths"],
                                                         new_v[:, None].astype(np.float64), max_context=4096)

    namespace = {"DecodePlan": __import__("paged_decode.runtime", fromlist=["DecodePlan"]).DecodePlan,
                 "torch": torch, "layout": layout, "table": table, "lengths": lengths, "q": q, "k": k, "v": v,
                 "q_step": q_step, "k_step": k_step, "v_step": v_step, "fill": fill, "steps": 3}
    exec(compile(block("torch.cuda.CUDAGraph()"), str(INTEGRATION), "exec"), namespace)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(namespace["plan"]._lengths.cpu().numpy(), host["lengths"])
    expected = fp64.dense_attention(host["q"], host["k"], host["v"], table, host["lengths"])
    assert_parity(namespace["out"].cpu().numpy(), expected, torch.float16)


def test_ctypes_snippet():
    announce("INTEGRATION ctypes call")
    layout, table, lengths = make_metadata(3, 32, 8, 128, 1000, 16, seed=11)
    qf, kf, vf = host_tensors(layout, dtype=np.float32, seed=12)
    largest = float(torch.finfo(torch.float8_e4m3fn).max)
    k_scale, v_scale = float(np.abs(kf).max()) / largest, float(np.abs(vf).max()) / largest
    q = torch.from_numpy(qf).bfloat16().cuda()
    k = (torch.from_numpy(kf) / k_scale).to(torch.float8_e4m3fn).cuda()
    v = (torch.from_numpy(vf) / v_scale).to(torch.float8_e4m3fn).cuda()
    namespace = {"lengths": lengths, "split_tokens": 256, "B": layout.batch, "Hq": layout.query_heads,
                 "Hkv": layout.kv_heads, "D": layout.head_dim, "T": layout.page_size, "W": table.shape[1],
                 "P": layout.physical_pages, "q": q, "k": k, "v": v, "k_scale": k_scale, "v_scale": v_scale,
                 "d_table": torch.from_numpy(table).cuda(), "d_lengths": torch.from_numpy(lengths).cuda()}
    exec(compile(block("lib.pd_decode_ex("), str(INTEGRATION), "exec"), namespace)
    torch.cuda.synchronize()
    exact = (q.double().cpu().numpy(), k.double().cpu().numpy() * k_scale, v.double().cpu().numpy() * v_scale)
    assert namespace["splits"] == math.ceil(int(lengths.max()) / 256)
    assert_parity(namespace["out"].cpu().numpy(), fp64.dense_attention(*exact, table, lengths), torch.float16)
