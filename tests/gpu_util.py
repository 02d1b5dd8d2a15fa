"""Helpers shared by the GPU test modules."""
import sys

import numpy as np
import pytest

try:
    import torch
except ImportError:  # pragma: no cover
    torch = None

# Parity bar: FP32 inputs within 1e-5 relative (elementwise, with a 1e-6
# absolute floor for outputs near zero); FP16 inputs within 2e-3 absolute.
# Every case also meets the reference's own 5e-4 gate (tests/test_cuda.py:31).
FP32_RTOL, FP32_ATOL = 1e-5, 1e-6
FP16_ATOL = 2e-3
REFERENCE_TOL = 5e-4


def require_gpu():
    if torch is None or not torch.cuda.is_available():
        pytest.skip("needs a GPU", allow_module_level=True)


def no_child_processes_after_gpu_init():
    """Skip a CPU test that starts a child process (a compiler, python) when
    this process has initialised the GPU: a program started from such a
    process can take the GPU runtime down with it."""
    torch_module = sys.modules.get("torch")
    if torch_module is not None and torch_module.cuda.is_initialized():
        pytest.skip("the GPU was initialised in this process; no child processes are started")


def announce(message):
    print(message, flush=True)
    sys.stdout.flush()


def assert_parity(actual, expected, dtype, reference_tol=REFERENCE_TOL):
    actual = np.asarray(actual, dtype=np.float64)
    assert np.isfinite(actual).all()
    if dtype in (np.float32, "float32") or (torch is not None and dtype == torch.float32):
        np.testing.assert_allclose(actual, expected, rtol=FP32_RTOL, atol=FP32_ATOL)
    else:
        np.testing.assert_allclose(actual, expected, rtol=0, atol=FP16_ATOL)
    if reference_tol is not None:
        np.testing.assert_allclose(actual, expected, rtol=reference_tol, atol=reference_tol)


def host(*tensors):
    return tuple(t.detach().cpu().numpy() for t in tensors)
