"""Host memory checks: the partition kernels' address map and the C restatement.

The reference ran compute-sanitizer memcheck over its GPU tests
(tools/gpu_acceptance.sh:4-15). Here the same question -- does any access
leave its buffer? -- is answered on the CPU:

* ``tests/address_audit.cpp`` walks every workgroup, wave, lane and load group
  of the partition launches, and every workgroup and lane of the merge
  launches that follow them (both merge kernels in every variant: serial and
  shared, plain and XCD-grouped rows, combined-quarter strides, short and
  long rounds, both column-chunk widths), for the measured workloads and the edge cases
  (lengths around page and partition boundaries, invalid page ids, uncommon
  head layouts, a 1M-token context in a 65536-wide table, pages above 4 GiB,
  work lists and rectangular grids with tail items under exact, low and zero
  length bounds, whole-row launches, full calls over the coarser partitions
  of large grids, shared-prefix items under true and stale prefix runs,
  including seeded random sharing patterns) through the
  same ``partition_map.h`` functions the kernels call, and checks every load,
  store and LDS access against its buffer, every live token against the page
  its table entry names, and that every live state slot is written exactly
  once; that every merge load, LDS weight and output store stays in its buffer,
  every output element is written once and every state a merge counts as
  live was written by its partition launch. It also walks the KV-cache append
  (explicit positions and the advancing variant) and the device CSR -> page
  table conversion over valid and malformed metadata. Each kernel family has
  a planted-mistake negative control (wrong reach, merge live count, append
  capacity, missing CSR indices bound, shared-prefix items without their page
  check) that the walk must report. It is
  compiled with AddressSanitizer and UndefinedBehaviorSanitizer.
* ``oracle/cpu_decode.c`` (the FP32 restatement the bench times) runs under
  the same sanitizers on ragged, empty-row, invalid-page-id and both-format
  cases through a small C driver.
"""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

from gpu_util import no_child_processes_after_gpu_init

REPO = Path(__file__).resolve().parent.parent
CSRC = REPO / "paged-decode-lab_amd" / "paged_decode" / "csrc"
SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer"]
ENV = {**os.environ, "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1"}


def compiler(name):
    no_child_processes_after_gpu_init()
    path = shutil.which(name)
    if path is None:
        pytest.skip(f"{name} not available")
    return path


@pytest.fixture(scope="module")
def audit_exe(tmp_path_factory):
    exe = tmp_path_factory.mktemp("audit") / "address_audit"
    subprocess.run([compiler("g++"), "-std=c++17", "-O1", "-g", "-Wall", "-Wno-unknown-pragmas", *SANITIZE,
                    f"-I{CSRC}", str(REPO / "tests" / "address_audit.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, text=True)
    return exe


def test_partition_address_map_stays_in_bounds(audit_exe):
    run = subprocess.run([str(audit_exe)], capture_output=True, text=True, timeout=600, env=ENV)
    assert run.returncode == 0, run.stdout[-4000:] + run.stderr[-4000:]
    assert ", 0 failures" in run.stdout
    # The walk covered the measured workloads and the compacted launches.
    for needle in ("llama3-8b B4 L4096 fp16", "ragged shared B16", "mqa B128", "long mha B1", "compact",
                   "rectangular+tails", "whole rows", "1M context", "pages above 4 GiB", "invalid page ids fp8",
                   "ragged shared B16 T32 split 128 bounds=exact coarse x8", "bounds=half coarse x4",
                   "long mha B1 Hq32/32 L32768 split 128 bounds=exact coarse x8",
                   "past reach B64 Hq32/8 D128 splits 3x256 L1000 bounds=exact coarse x2"):
        assert needle in run.stdout, needle
    # The XCD-grouped grid is chosen for the measured uniform workloads and the
    # shapes of tests/test_gpu_xcd_grid.py under bounds, and not without them;
    # with eight head groups per sequence only the merge is XCD-grouped (the
    # plain grids already are), bounds or not.
    assert "xcd merge" in "\n".join(line for line in run.stdout.splitlines()
                                     if line.startswith("long mha B1 Hq32/32 L32768 split 1024 "))
    lines = run.stdout.splitlines()
    launches = [line for line in lines if " grid " in line]  # partition launches (merge lines say "merge")
    for name in ("llama3-8b B4 L4096 fp16", "llama3-8b B4 L4096 fp8", "xcd gqa4 B8 Hq32/8 D128 L1024 split 128 fp16",
                 "xcd gqa4 B8 Hq32/8 D128 L1024 split 128 fp8", "xcd mqa B64 Hq16/1 D64 L1024 split 256 fp16",
                 "xcd mha B2 Hq16/16 D128 L2048 split 256 fp16", "xcd fp32 B8 Hq16/8 D64 L1024 split 128",
                 "xcd llama3-8b B4 L4096 reserve x4", "xcd mqa B128 Hq16/1 D64 L1024 reserve x2"):
        exact = [line for line in launches if line.startswith((name + " bounds=exact ", name + " bounds=half "))]
        plain = [line for line in launches if line.startswith(name + " ") and "bounds=" not in line]
        assert len(exact) >= 2 and all("xcd-grouped" in line or "xcd merge" in line for line in exact), name
        assert plain and not any("xcd-grouped" in line for line in plain), name
    # Every merge kernel variant was walked, for staged and full calls.
    merges = [line for line in lines if " merge " in line and line.rstrip().endswith("ok")]
    for variant in ("serial:rows", "shared:rows", "rows/xcd", "cols/NB8/CH64", "cols/NB32/CH64", "cols/NB8/CH32/xcd",
                    "cols/NB32/CH32/xcd", "shared:cols/NB32", "stride2", "stride4"):
        assert any(variant in line for line in merges), variant
    assert any("[stage]" in line for line in merges) and any("[call]" in line for line in merges)
    summary = lines[-1]
    assert " merge launches, " in summary and " appends, " in summary and " csr conversions, " in summary
    assert any(line.startswith("append") and "append+advance" in line for line in lines)
    assert any(line.startswith("csr list past the indices end") and "1 of 2 rows rejected" in line for line in lines)
    # Shared-prefix items were walked for every tile width that takes them
    # (MHA: 16 members, GQA 4: 4, GQA 8: 2), with several sharing classes, at
    # the item cap, with members shorter on the device than their bounds, and
    # in the full call's coarser partitions; never without bounds or for FP32.
    shared = [line for line in launches if "shared-prefix items" in line]
    for name in ("prefix mha B24 Hq8/8 D64 T16 split 64 prefix runs bounds=exact",
                 "prefix gqa8 B6 Hq16/2 D128 T16 split 64 prefix runs bounds=exact",
                 "prefix two classes B16 Hq32/8 D128 T32 split 128 prefix runs bounds=exact",
                 "prefix two classes B16 Hq32/8 D128 T32 split 128 prefix runs lengths below bounds",
                 "prefix padded rows B24 Hq8/8 D64 T16 split 64 prefix runs bounds=exact",
                 "prefix padded rows B32 Hq32/8 D128 T16 split 256 prefix runs bounds=exact",
                 "prefix samples B16 Hq32/8 D128 T16 L4096 split 256 prefix runs bounds=exact"):
        assert any(line.startswith(name + " ") for line in shared), name
    assert any(line.startswith("prefix cap ") and ", 128 shared-prefix items" in line for line in shared)
    # The seeded random sharing patterns formed items on many launches.
    assert sum(1 for line in shared if line.startswith("prefix random ")) >= 20
    # Runs that claim more than the table shares (stale runs) stay correct:
    # the page check sends the differing members to passes of their own.
    assert any(" prefix runs stale bounds=exact " in line and " own passes)" in line for line in shared)
    assert not any(" own passes)" in line for line in shared if " stale " not in line and "bounds=half" not in line)
    # Equal lengths with a shared prompt: the rectangular grid became a work
    # list, and the full call took half the coarse split that fills the device
    # without items (x4 for this batch), where the items pay.
    assert any(line.startswith("prefix samples B16 Hq32/8 D128 T16 L4096 split 256 prefix runs bounds=exact ")
               and " compact," in line for line in shared)
    assert any(line.startswith("prefix samples B16 Hq32/8 D128 T16 L4096 split 256 prefix runs bounds=exact "
                               "coarse x2 [call] mfma") and " compact," in line for line in shared)
    own_passes = int(summary.split(" shared-prefix own passes")[0].rsplit(", ", 1)[1])
    assert own_passes > 0, summary
    assert any("coarse x" in line and "[call]" in line for line in shared)
    assert not any("bounds=zero" in line or " fp32 " in line for line in shared)


@pytest.mark.parametrize("plant,message", [
    ("--plant-reach", "wave range [768, 896)"),
    ("--plant-merge-live", "that the partition launch did not write"),
    ("--plant-append", "append reads table entry"),
    ("--plant-csr", "indices read 6 of 6"),
    ("--plant-prefix", "the item reads page"),
])
def test_address_audit_flags_planted_mistakes(audit_exe, plant, message):
    """Negative controls: launch parameters with one mistake planted (lengths
    clamped to the table instead of the caller's partitions; a merge live
    count one partition too long; an append capacity one page past the table;
    a CSR conversion without its bound on the indices read; shared-prefix
    items that trust stale runs, without the kernel's page check). Each walk
    must report the accesses the mistake causes."""
    run = subprocess.run([str(audit_exe), plant], capture_output=True, text=True, timeout=300, env=ENV)
    assert run.returncode == 1, run.stdout[-4000:] + run.stderr[-4000:]
    assert "FAIL" in run.stderr and message in run.stderr


CPU_DRIVER = r"""
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

int pd_cpu_decode(const void* q, const void* k, const void* v, int dtype, const int32_t* table,
                  const int32_t* lengths, float* out, int batch, int q_heads, int kv_heads, int head_dim,
                  int page_size, int table_width, int physical_pages, int split_tokens, int threads);

static uint32_t state = 12345u;
static float next_value(void) {
    state = state * 1664525u + 1013904223u;
    return (float)((state >> 8) & 0xFFFF) / 32768.0f - 1.0f;
}

/* One case: exact-size heap buffers, so any out-of-bounds access trips ASan. */
static int run_case(int dtype, int batch, int hq, int hkv, int dim, int page, int width, int pages,
                    const int32_t* lengths, int poison_ids, int split) {
    size_t elem = dtype == 0 ? 4 : 2;
    size_t qn = (size_t)batch * hq * dim, kn = (size_t)pages * page * hkv * dim;
    unsigned char* q = malloc(qn * elem);
    unsigned char* k = malloc(kn * elem);
    unsigned char* v = malloc(kn * elem);
    int32_t* table = malloc(sizeof(int32_t) * batch * width);
    int32_t* lens = malloc(sizeof(int32_t) * batch);
    float* out = malloc(sizeof(float) * qn);
    for (size_t i = 0; i < qn * elem / 2; ++i) ((uint16_t*)q)[i] = dtype == 0 ? 0 : 0x3C00;
    if (dtype == 0) for (size_t i = 0; i < qn; ++i) ((float*)q)[i] = next_value();
    if (dtype == 0) for (size_t i = 0; i < kn; ++i) { ((float*)k)[i] = next_value(); ((float*)v)[i] = next_value(); }
    else for (size_t i = 0; i < kn; ++i) { ((uint16_t*)k)[i] = 0x3800; ((uint16_t*)v)[i] = 0x3400; }
    for (int i = 0; i < batch * width; ++i) table[i] = (i * 7) % pages;
    if (poison_ids) { table[0] = -1; table[width + 1] = pages; table[2 * width] = 0x7FFFFFFF; }
    memcpy(lens, lengths, sizeof(int32_t) * batch);
    int status = pd_cpu_decode(q, k, v, dtype, table, lens, out, batch, hq, hkv, dim, page, width, pages, split, 2);
    for (size_t i = 0; status == 0 && i < qn; ++i) if (!isfinite(out[i])) status = 9;
    free(q); free(k); free(v); free(table); free(lens); free(out);
    return status;
}

int main(void) {
    const int32_t ragged[4] = {100, 0, 256, 17};
    const int32_t beyond[4] = {1 << 20, 1, 33, 255};   /* first length past the table: clamped */
    int failures = 0;
    for (int dtype = 0; dtype < 2; ++dtype) {
        for (int split = 1; split <= 256; split *= 16) {
            failures += run_case(dtype, 4, 8, 2, 64, 16, 16, 64, ragged, 0, split) != 0;
            failures += run_case(dtype, 4, 8, 2, 128, 32, 8, 32, beyond, 1, split) != 0;
            failures += run_case(dtype, 4, 12, 4, 64, 16, 16, 64, ragged, 1, split) != 0;
        }
    }
    printf("cpu restatement sanitizer cases: %d failures\n", failures);
    return failures != 0;
}
"""


def test_cpu_restatement_stays_in_bounds(tmp_path):
    driver = tmp_path / "driver.c"
    driver.write_text(CPU_DRIVER)
    exe = tmp_path / "cpu_driver"
    subprocess.run([compiler("gcc"), "-O1", "-g", "-march=x86-64-v3", "-fopenmp", *SANITIZE,
                    str(REPO / "oracle" / "cpu_decode.c"), str(driver), "-o", str(exe), "-lm"],
                   check=True, capture_output=True, text=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300, env=ENV)
    assert run.returncode == 0, run.stdout[-4000:] + run.stderr[-4000:]
    assert "0 failures" in run.stdout
