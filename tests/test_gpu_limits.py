"""The supported limits: a 1M-token context and a K/V cache above 4 GiB.

* One sequence of exactly 1,048,576 tokens with a page table 65,536 wide
  (both limits of the plan), split 256: 16,384 states per row, merged in many
  load rounds (the shared merge falls back to serial above 4096 states).
* A cache of more than 4 GiB per tensor whose live pages sit at its top, so
  page offsets need 64-bit address arithmetic. Only the live pages are filled;
  the oracle runs on a compacted copy of them with the table relabelled.
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("merge", ["serial", "shared"])
def test_context_of_one_million_tokens(merge):
    announce(f"1M-token context merge={merge}")
    context, page, width = 1 << 20, 16, 1 << 16
    layout = Layout(1, 8, 1, 64, page, width)
    rng = np.random.default_rng(21)
    table = rng.permutation(width).astype(np.int32)[None, :]
    lengths = np.array([context], dtype=np.int32)
    q = rng.standard_normal((1, 8, 64), dtype=np.float32).astype(np.float16)
    k = rng.standard_normal((width, page, 1, 64), dtype=np.float32).astype(np.float16)
    v = rng.standard_normal((width, page, 1, 64), dtype=np.float32).astype(np.float16)
    plan = DecodePlan(layout, table, lengths, split_tokens=256, merge=merge)
    assert plan.splits == 4096
    assert plan.merge_implementation == ("serial" if merge == "serial" else "serial_fallback")
    out = plan.run(*(torch.from_numpy(x).cuda() for x in (q, k, v))).cpu().numpy()
    assert_parity(out, dense_attention(q, k, v, table, lengths), torch.float16)


def test_cache_larger_than_4gib():
    announce("cache > 4 GiB, live pages at its top")
    page, kv_heads, dim = 16, 8, 128
    page_bytes = page * kv_heads * dim * 2
    pages = (5 << 30) // page_bytes                      # 5 GiB per tensor
    live = 64
    layout = Layout(2, 32, kv_heads, dim, page, pages)
    rng = np.random.default_rng(8)
    top = np.arange(pages - live, pages, dtype=np.int64)
    table = rng.permutation(top).reshape(2, live // 2).astype(np.int32)
    lengths = np.array([live // 2 * page, live // 2 * page - 9], dtype=np.int32)
    k = torch.empty((pages, page, kv_heads, dim), dtype=torch.float16, device="cuda")
    v = torch.empty_like(k)
    k_live = rng.standard_normal((live, page, kv_heads, dim), dtype=np.float32).astype(np.float16)
    v_live = rng.standard_normal((live, page, kv_heads, dim), dtype=np.float32).astype(np.float16)
    k[pages - live:] = torch.from_numpy(k_live).cuda()
    v[pages - live:] = torch.from_numpy(v_live).cuda()
    q = rng.standard_normal((2, 32, dim), dtype=np.float32).astype(np.float16)
    plan = DecodePlan(layout, table, lengths, split_tokens=128)
    out = plan.run(torch.from_numpy(q).cuda(), k, v).cpu().numpy()
    compact = (table - (pages - live)).astype(np.int32)  # the same pages, relabelled into the compact copy
    assert_parity(out, dense_attention(q, k_live, v_live, compact, lengths), torch.float16)
    assert (int(table.max()) + 1) * page_bytes > (4 << 30)
