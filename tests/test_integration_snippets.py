"""The C snippets of INTEGRATION.md compile against include/paged_decode.h.

Each ```c block of the document is taken as it stands: its #include lines go
to the top of a translation unit, its statements into one function whose
parameters are the buffers and sizes the snippets name, and gcc checks the
unit (-fsyntax-only, warnings as errors for implicit declarations and
mismatched argument types). A snippet that drifts from the header's
signatures fails here.
"""
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from gpu_util import no_child_processes_after_gpu_init

REPO = Path(__file__).resolve().parent.parent
INTEGRATION = REPO / "INTEGRATION.md"

PRELUDE = """#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
"""
PARAMS = ("const void* q, const void* k, const void* v, const int32_t* table, const int32_t* lengths, "
          "const int32_t* host_table, const int32_t* host_lengths, float* ws_num, float* ws_stats, float* out, "
          "int B, int Hq, int Hkv, int D, int T, int W, int P, int splits, int split_tokens, void* stream")


def c_blocks():
    return re.findall(r"```c\n(.*?)```", INTEGRATION.read_text(), flags=re.S)


def test_integration_has_c_snippets():
    blocks = c_blocks()
    assert len(blocks) >= 2
    assert any("pd_decode_prefix" in block and "pd_prefix_runs" in block for block in blocks)


def test_c_snippets_compile(tmp_path):
    no_child_processes_after_gpu_init()
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    includes, body = [], []
    for block in c_blocks():
        for line in block.splitlines():
            (includes if line.startswith("#include") else body).append(line)
    source = PRELUDE + "\n".join(includes) + f"\n\nint snippets({PARAMS}) {{\n" + "\n".join(body) + \
        "\n    return rc;\n}\n"
    unit = tmp_path / "snippets.c"
    unit.write_text(source)
    run = subprocess.run([gcc, "-std=c11", "-fsyntax-only", "-Wall", "-Werror=implicit-function-declaration",
                          "-Werror=incompatible-pointer-types", "-Werror=int-conversion", "-Wno-unused-variable",
                          f"-I{REPO / 'include'}", str(unit)], capture_output=True, text=True)
    assert run.returncode == 0, source + "\n" + run.stderr
