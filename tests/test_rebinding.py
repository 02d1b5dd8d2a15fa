"""The reference-side rebinding documented in INTEGRATION.md loads, from
inside a package that owns the name ``paged_decode``.

A stand-in package named ``paged_decode`` (none of the reference's files is
imported) gets a ``runtime.py`` made of the reference module's own imports
(``runtime.py:1-6``) and the replacement ``load_extension()`` extracted from
INTEGRATION.md. A separate Python process, whose import path holds only that
stand-in, calls it: the name collision the reference package creates
(``src/paged_decode/__init__.py:1-3``) is then exactly as a maintainer meets
it. The GPU side of the same binding (the reference's ten-argument call
through the module loaded this way) is in tests/test_gpu_reference_call.py.
"""
import json
import os
import subprocess
import sys

import pytest

import rebinding
from gpu_util import no_child_processes_after_gpu_init
from paged_decode import _build, cabi

STAND_IN_RUNTIME = '''"""Stand-in for the reference's runtime module: its imports, then the rebinding."""
from functools import lru_cache
from pathlib import Path
import math
import torch

'''

PROBE = '''
import json, sys
import paged_decode, paged_decode.runtime as runtime
extension = runtime.load_extension()
print(json.dumps({"package": paged_decode.__file__, "version": paged_decode.__version__,
                  "abi": extension.header_abi_version(), "library_abi": extension.abi_version(),
                  "has_decode": hasattr(extension, "decode"), "module": extension.__name__,
                  "cached": runtime.load_extension() is extension}))
'''


def test_snippet_is_the_documented_function():
    source = rebinding.snippet()
    assert "def load_extension():" in source and "@lru_cache(maxsize=1)" in source
    assert "spec_from_file_location" in source
    assert 'import_module("paged_decode._C")' not in source


def test_documented_rebinding_loads_inside_a_package_named_paged_decode(tmp_path):
    no_child_processes_after_gpu_init()
    if not _build.built():
        pytest.skip("native libraries not built")
    package = tmp_path / "reference_src" / "paged_decode"
    package.mkdir(parents=True)
    (package / "__init__.py").write_text('"""Stand-in for the reference package."""\n\n__version__ = "0.2.0"\n')
    (package / "runtime.py").write_text(STAND_IN_RUNTIME + rebinding.snippet())
    env = {k: v for k, v in os.environ.items() if k != "PYTHONPATH"}
    env["PYTHONPATH"] = str(package.parent)
    env["PAGED_DECODE_AMD"] = str(rebinding.PACKAGE_ROOT)
    run = subprocess.run([sys.executable, "-c", PROBE], capture_output=True, text=True, timeout=300, env=env,
                         cwd=tmp_path)
    assert run.returncode == 0, run.stdout[-3000:] + run.stderr[-3000:]
    result = json.loads(run.stdout.strip().splitlines()[-1])
    assert result["package"] == str(package / "__init__.py") and result["version"] == "0.2.0"
    assert result["abi"] == result["library_abi"] == cabi.PD_ABI_VERSION
    assert result["has_decode"] and result["cached"]
    assert result["module"] == "paged_decode_amd._C"


def test_documented_rebinding_reports_a_missing_build(tmp_path):
    """Pointed at a directory without the libraries, the loader raises ImportError."""
    with pytest.raises(ImportError):
        rebinding.load_as_documented(tmp_path)
