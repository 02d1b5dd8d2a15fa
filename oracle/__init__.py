"""Reference restatements used ONLY to check and baseline the decode operator.

This directory is test infrastructure. Only ``tests/``, ``__graft_entry__.smoke()``
and the CPU-baseline leg of ``bench.py`` import, call or load anything here; the
``paged_decode`` package never does, and its GPU path fails loudly instead of
falling back to CPU code.

* ``fp64.py`` -- NumPy FP64 oracle (dense softmax attention over the paged
  cache, the online-softmax recurrence and the max-corrected merge), restating
  reference ``src/paged_decode/oracle.py:50-117`` and ``docs/DESIGN.md:5-65``.
* ``cpu_decode.c`` -- multithreaded FP32 split-K paged decode in C with the GPU
  path's semantics (empty rows give zeros, the ``l > 0`` merge guard, the
  page-id guard). It is the timed CPU baseline and a second cross-check.
* ``cpu.py`` -- ctypes loader for the C restatement (built by ``Makefile``).

Pinning (what fixes each function independently of its own formula) is listed
in the module docstrings and exercised by ``tests/test_oracle.py``.
"""
