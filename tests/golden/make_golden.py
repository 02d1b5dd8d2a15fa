"""Regenerate the committed fixtures in this directory.

* ``recorded_metadata.json`` -- sequence lengths that the reference's own
  benchmark reports recorded for ``make_metadata(..., seed=123)`` (read as JSON
  data from ``results/2026-10-31-t4/*.json`` under the reference checkout; no
  reference code is imported or run). They pin ``paged_decode.workload.make_metadata``.
* ``expected_outputs.npz`` -- FP64 oracle outputs for small seeded inputs
  (inputs are regenerated from their seeds by NumPy's PCG64, which is stable
  across platforms), plus SHA-256 digests of the inputs so a changed generator
  is detected before outputs are compared.

Run from the repository root: ``python tests/golden/make_golden.py [REFERENCE_ROOT]``.
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "paged-decode-lab_amd"))

from oracle import fp64  # noqa: E402
from paged_decode.workload import make_workload  # noqa: E402
from paged_decode.layout import Layout  # noqa: E402
from paged_decode.workload import host_tensors  # noqa: E402


def recorded_metadata(reference_root):
    cases = []
    for path in sorted((Path(reference_root) / "results" / "2026-10-31-t4").glob("*.json")):
        report = json.loads(path.read_text())
        config = report.get("configuration", {})
        workload = report.get("workload", {})
        if "lengths" not in workload:
            continue
        cases.append({
            "source": f"results/2026-10-31-t4/{path.name}",
            "batch": config["batch"], "heads": config["heads"], "kv_heads": config["kv_heads"],
            "dim": config["dim"], "context": config["context"], "page_size": config["page_size"],
            "seed": config["seed"], "uniform": config.get("uniform", False),
            "lengths": workload["lengths"],
            "physical_pages": workload["physical_pages"],
        })
    return cases


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


SMALL_CASES = {
    # name: (layout args, lengths, table seed, value seed, dtype)
    "gqa4_f32_ragged": ((4, 8, 2, 64, 16, 32), [0, 1, 17, 127], 5, 11, np.float32),
    "gqa4_f16_ragged": ((4, 8, 2, 128, 32, 32), [0, 1, 33, 127], 6, 12, np.float16),
    "mqa_f16_shared_pages": ((2, 8, 1, 128, 16, 4), [64, 37], None, 13, np.float16),
}


def small_case_inputs(name):
    layout_args, lengths, table_seed, value_seed, dtype = SMALL_CASES[name]
    layout = Layout(*layout_args)
    lengths = np.array(lengths, dtype=np.int32)
    width = max(1, (int(lengths.max()) + layout.page_size - 1) // layout.page_size)
    if table_seed is None:
        table = np.array([[2, 0, 1, 3], [2, 0, 1, 3]], dtype=np.int32)[:, :width]
    else:
        table = np.random.default_rng(table_seed).permutation(layout.physical_pages)[
            :layout.batch * width].reshape(layout.batch, width).astype(np.int32)
    for row, length in enumerate(lengths):
        table[row, (int(length) + layout.page_size - 1) // layout.page_size:] = -1
    q, k, v = host_tensors(layout, dtype=dtype, seed=value_seed)
    return layout, table, lengths, q, k, v


def expected_outputs():
    out = {}
    w = make_workload("fp32_b2_ragged")
    q, k, v = w.host_tensors()
    out["fp32_b2_ragged/out"] = fp64.dense_attention(q, k, v, w.table, w.lengths)
    out["fp32_b2_ragged/digest"] = np.array(digest(q, k, v, w.table, w.lengths))
    for name in SMALL_CASES:
        layout, table, lengths, q, k, v = small_case_inputs(name)
        out[f"{name}/out"] = fp64.dense_attention(q, k, v, table, lengths)
        out[f"{name}/digest"] = np.array(digest(q, k, v, table, lengths))
    return out


def main():
    reference_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    if Path(reference_root).exists():
        cases = recorded_metadata(reference_root)
        (HERE / "recorded_metadata.json").write_text(json.dumps(cases, indent=1) + "\n")
        print(f"recorded_metadata.json: {len(cases)} cases")
    np.savez_compressed(HERE / "expected_outputs.npz", **expected_outputs())
    print("expected_outputs.npz written")


if __name__ == "__main__":
    main()
