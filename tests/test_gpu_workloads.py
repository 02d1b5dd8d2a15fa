"""GPU parity on the named decode workloads and full-size properties.

Every workload is compared with the FP64 oracle at its real size (the oracle
finishes in seconds on these shapes). Size-independent properties add checks
that do not depend on the oracle at all: bitwise invariance under physical
page relabelling, agreement across split sizes, GQA equal to MHA over
repeated KV heads, and identical rows for identical sequences.
"""
import numpy as np
import pytest

from gpu_util import announce, assert_parity, host, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.runtime import DecodePlan  # noqa: E402
from paged_decode.workload import WORKLOAD_NAMES, make_workload  # noqa: E402

pytestmark = pytest.mark.gpu


def device_inputs(w):
    return tuple(torch.from_numpy(x).cuda() for x in w.host_tensors())


@pytest.mark.parametrize("name", WORKLOAD_NAMES)
def test_named_workload_parity(name):
    w = make_workload(name)
    q, k, v, k_scale, v_scale = w.tensors("cuda")
    expected = dense_attention(*w.host_tensors(), w.table, w.lengths)
    splits = w.split_sweep or (w.split_tokens,)
    for split in splits:
        for merge in ("serial", "shared"):
            announce(f"workload {name} split={split} merge={merge}")
            plan = DecodePlan(w.layout, w.table, w.lengths, split_tokens=split, merge=merge)
            actual = plan.run(q, k, v, k_scale=k_scale, v_scale=v_scale).cpu().numpy()
            assert_parity(actual, expected, w.dtype if w.native else torch.float16)
    empty = w.lengths == 0
    if empty.any():
        np.testing.assert_array_equal(actual[empty], 0.0)


def test_page_relabelling_is_bitwise_invisible():
    w = make_workload("llama3_8b_b4_l4096")
    q, k, v = device_inputs(w)
    plan = DecodePlan(w.layout, w.table, w.lengths, split_tokens=w.split_tokens)
    announce("relabel: original")
    base = plan.run(q, k, v).clone()
    perm = np.random.default_rng(77).permutation(w.layout.physical_pages)
    dest = torch.from_numpy(perm).cuda()
    k2, v2 = torch.empty_like(k), torch.empty_like(v)
    k2[dest] = k
    v2[dest] = v
    table2 = perm[w.table].astype(np.int32)
    plan2 = DecodePlan(w.layout, table2, w.lengths, split_tokens=w.split_tokens)
    announce("relabel: permuted")
    torch.testing.assert_close(plan2.run(q, k2, v2), base, rtol=0, atol=0)


def test_split_sizes_agree_at_long_context():
    w = make_workload("long_mha_b1_l32768")
    q, k, v = device_inputs(w)
    outs = []
    for split in (64, 128, 256, 512, 1024, 4096, 32768):
        announce(f"split sweep {split}")
        plan = DecodePlan(w.layout, w.table, w.lengths, split_tokens=split)
        outs.append(plan.run(q, k, v).cpu().numpy())
    for out in outs[1:]:
        np.testing.assert_allclose(out, outs[0], rtol=0, atol=1e-4)


def test_gqa_equals_mha_over_repeated_kv_heads():
    w = make_workload("llama3_8b_b4_l4096")
    q, k, v = device_inputs(w)
    plan = DecodePlan(w.layout, w.table, w.lengths, split_tokens=w.split_tokens)
    announce("gqa")
    gqa = plan.run(q, k, v).clone()
    L = w.layout
    mha_layout = Layout(L.batch, L.query_heads, L.query_heads, L.head_dim, L.page_size, L.physical_pages)
    k_mha = k.repeat_interleave(L.group, dim=2).contiguous()
    v_mha = v.repeat_interleave(L.group, dim=2).contiguous()
    plan_mha = DecodePlan(mha_layout, w.table, w.lengths, split_tokens=w.split_tokens)
    announce("mha")
    torch.testing.assert_close(plan_mha.run(q, k_mha, v_mha), gqa, rtol=0, atol=2e-6)


def test_identical_sequences_give_identical_rows():
    w = make_workload("mqa_b128_l1024")
    q, k, v = device_inputs(w)
    table = np.repeat(w.table[:1], w.layout.batch, axis=0)
    q_same = q[:1].expand_as(q).contiguous()
    plan = DecodePlan(w.layout, table, w.lengths, split_tokens=w.split_tokens)
    announce("identical rows")
    out = plan.run(q_same, k, v)
    torch.testing.assert_close(out, out[:1].expand_as(out), rtol=0, atol=0)


def test_merge_variants_agree():
    w = make_workload("mqa_b128_l1024")
    q, k, v = device_inputs(w)
    outs = {}
    for merge in ("serial", "shared"):
        announce(f"merge variant {merge}")
        outs[merge] = DecodePlan(w.layout, w.table, w.lengths, split_tokens=w.split_tokens,
                                 merge=merge).run(q, k, v).clone()
    torch.testing.assert_close(outs["shared"], outs["serial"], rtol=1e-6, atol=1e-6)
