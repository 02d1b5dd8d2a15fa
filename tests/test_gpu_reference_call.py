"""The reference's own call into the extension, against the FP64 oracle.

A maintainer who rebinds the reference's ``load_extension()`` to this build's
``_C`` module keeps the reference's ``DecodePlan``: it allocates
``numerator [B, Hq, 4S, D]``, ``stats [B, Hq, 4S, 2]`` and ``out`` with
``torch.empty`` (reference ``src/paged_decode/runtime.py:64-68``, S from the
longest sequence, ``runtime.py:46-49``) and calls ``decode`` with exactly ten
positional arguments (``runtime.py:88-89``, ``bindings.cpp:3-9``): no scales,
no hints. These tests make that call, on the FP32 oracle case and the
Llama-3-8B decode shape, for both merge modes, and the reference's
shared-merge bound (``decode.cu:234-235``) as a ``RuntimeError``. The
extension is reached two ways: through this package's ``load_extension``,
and through the replacement ``load_extension()`` INTEGRATION.md gives for
the reference's ``runtime.py`` (loaded by file location, as it must be
inside a package that owns the name ``paged_decode``).
"""
import math

import numpy as np
import pytest

from gpu_util import announce, assert_parity, require_gpu

require_gpu()

import torch  # noqa: E402

import rebinding  # noqa: E402
from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode import cabi  # noqa: E402
from paged_decode.runtime import load_extension  # noqa: E402
from paged_decode.workload import make_workload  # noqa: E402

pytestmark = pytest.mark.gpu


def reference_buffers(layout, lengths, split_tokens, device):
    """The reference plan's workspace and output, allocated as it allocates them."""
    max_context = int(np.asarray(lengths).max(initial=0))
    splits = max(1, math.ceil(max_context / split_tokens))
    shape = (layout.batch, layout.query_heads, splits * 4)
    numerator = torch.empty((*shape, layout.head_dim), device=device, dtype=torch.float32)
    stats = torch.empty((*shape, 2), device=device, dtype=torch.float32)
    out = torch.empty((layout.batch, layout.query_heads, layout.head_dim), dtype=torch.float32, device=device)
    return numerator, stats, out


BINDINGS = {"package": load_extension, "documented": rebinding.load_as_documented}


@pytest.mark.parametrize("binding", sorted(BINDINGS))
@pytest.mark.parametrize("name", ["fp32_b2_ragged", "llama3_8b_b4_l4096"])
@pytest.mark.parametrize("merge_mode", [0, 1])
def test_reference_ten_argument_call(name, merge_mode, binding):
    announce(f"reference decode(...) call: workload {name} merge_mode={merge_mode} binding={binding}")
    w = make_workload(name)
    device = torch.device("cuda", torch.cuda.current_device())
    host = w.host_tensors()
    q, k, v = (torch.from_numpy(x).to(device) for x in host)
    table = torch.tensor(w.table, device=device)
    lengths = torch.tensor(w.lengths, device=device)
    numerator, stats, out = reference_buffers(w.layout, w.lengths, w.split_tokens, device)
    extension = BINDINGS[binding]()
    if binding == "documented":
        assert extension.__name__ == "paged_decode_amd._C" and extension.header_abi_version() == cabi.PD_ABI_VERSION
    result = extension.decode(q, k, v, table, lengths, numerator, stats, out, w.split_tokens, merge_mode)
    assert result is None
    expected = dense_attention(*host, w.table, w.lengths)
    assert_parity(out.cpu().numpy(), expected, w.dtype)
    # A second call on the same buffers (the reference's replay) gives the same bits.
    first = out.clone()
    extension.decode(q, k, v, table, lengths, numerator, stats, out, w.split_tokens, merge_mode)
    torch.cuda.synchronize()
    assert torch.equal(out, first)


def test_reference_call_rejects_shared_merge_past_its_bound():
    """4S > 4096 states with merge_mode 1 is a RuntimeError before any launch, as at reference
    decode.cu:234-235; the same buffers with merge_mode 0 decode correctly."""
    announce("reference decode(...) call: shared merge beyond 4096 states")
    w = make_workload("fp32_b2_ragged")
    device = torch.device("cuda", torch.cuda.current_device())
    host = w.host_tensors()
    q, k, v = (torch.from_numpy(x).to(device) for x in host)
    table = torch.tensor(w.table, device=device)
    lengths = torch.tensor(w.lengths, device=device)
    # One token per split: the reference plan for these lengths (S = 256,
    # 1024 states) is within the bound; buffers for 1025 tokens of context
    # (S = 1025, 4100 states) are not.
    split_tokens = 1
    lengths_1025 = np.array([100, 1025], dtype=np.int32)
    numerator, stats, out = reference_buffers(w.layout, lengths_1025, split_tokens, device)
    assert numerator.shape[2] == 4100
    out.fill_(float("nan"))
    extension = load_extension()
    with pytest.raises(RuntimeError, match="4096"):
        extension.decode(q, k, v, table, lengths, numerator, stats, out, split_tokens, 1)
    torch.cuda.synchronize()
    assert torch.isnan(out).all()
    extension.decode(q, k, v, table, lengths, numerator, stats, out, split_tokens, 0)
    assert_parity(out.cpu().numpy(), dense_attention(*host, w.table, w.lengths), w.dtype)
