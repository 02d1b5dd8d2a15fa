"""The dense PyTorch comparison baselines agree with the FP64 oracle (reference
tests/test_reference.py restated on the GPU); empty rows give zeros."""
import numpy as np
import pytest

from gpu_util import announce, require_gpu

require_gpu()

import torch  # noqa: E402

from oracle.fp64 import dense_attention  # noqa: E402
from paged_decode.baselines import dense_decode  # noqa: E402
from paged_decode.workload import make_workload  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["fp32_b2_ragged", "ragged_shared_b16"])
@pytest.mark.parametrize("kind", ["sdpa", "eager"])
def test_dense_baselines_match_oracle(name, kind):
    announce(f"baseline {kind} {name}")
    w = make_workload(name)
    qh, kh, vh = w.host_tensors()
    q, k, v = (torch.from_numpy(x).cuda() for x in (qh, kh, vh))
    table = torch.from_numpy(w.table).cuda()
    lengths = torch.from_numpy(w.lengths).cuda()
    out = dense_decode(q, k, v, table, lengths, kind=kind).float().cpu().numpy()
    expected = dense_attention(qh, kh, vh, w.table, w.lengths)
    empty = w.lengths == 0
    if kind == "eager":
        np.testing.assert_array_equal(out[empty], 0.0)
    live = ~empty
    np.testing.assert_allclose(out[live], expected[live], atol=3e-3, rtol=0)
