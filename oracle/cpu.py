"""ctypes loader for the C FP32 restatement in ``cpu_decode.c`` (test infrastructure).

``decode`` takes host NumPy arrays (float16 or float32 q/k/v, int32 metadata)
and returns the FP32 ``[B, Hq, D]`` output. Built by ``make -C oracle``.
"""
import ctypes
import os
import subprocess
import sys
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
LIBRARY = _HERE / "libpd_cpu.so"
_lib = None


def _gpu_initialised():
    torch = sys.modules.get("torch")
    return torch is not None and torch.cuda.is_initialized()


def build(verbose=False):
    """Compile ``libpd_cpu.so`` next to its source. Refused (RuntimeError) in a
    process that has initialised the GPU, which must not start a child
    process (here ``make`` and the compiler): build it beforehand."""
    if _gpu_initialised():
        raise RuntimeError("building oracle/libpd_cpu.so would start make from a process that has initialised the "
                           "GPU; build it first (make -C oracle) and restart")
    result = subprocess.run(["make", "-B", "-C", str(_HERE), "libpd_cpu.so"],
                            capture_output=not verbose, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"building the C restatement failed:\n{result.stdout}\n{result.stderr}")


def library():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        fn = lib.pd_cpu_decode
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.c_void_p] * 3 + [ctypes.c_int] + [ctypes.c_void_p] * 3 + [ctypes.c_int] * 9
        _lib = lib
    return _lib


def default_threads():
    """Host cores this process may run on."""
    return len(os.sched_getaffinity(0))


def decode(q, k, v, table, lengths, split_tokens=256, threads=None):
    """FP32 split-K decode of host arrays; returns ``float32 [B, Hq, D]``."""
    q = np.ascontiguousarray(q)
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    if q.dtype != k.dtype or q.dtype != v.dtype or q.dtype not in (np.float16, np.float32):
        raise TypeError("q/k/v must share float16 or float32 dtype")
    table = np.ascontiguousarray(table, dtype=np.int32)
    lengths = np.ascontiguousarray(lengths, dtype=np.int32)
    batch, heads, dim = q.shape
    pages, page_size, kv_heads, _ = k.shape
    out = np.empty((batch, heads, dim), dtype=np.float32)
    status = library().pd_cpu_decode(
        q.ctypes.data, k.ctypes.data, v.ctypes.data, 1 if q.dtype == np.float16 else 0,
        table.ctypes.data, lengths.ctypes.data, out.ctypes.data,
        batch, heads, kv_heads, dim, page_size, table.shape[1], pages, int(split_tokens),
        int(threads or default_threads()))
    if status != 0:
        raise ValueError(f"pd_cpu_decode failed with status {status}")
    return out
