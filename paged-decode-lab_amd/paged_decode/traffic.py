"""HBM bytes per partition launch, from two ``rocprofv3 --pmc`` passes.

``run`` is the program the counter passes profile: it builds a DecodePlan for a
named workload, replicates K/V into buffer sets covering >= 2 GiB (so no
launch is served from the 256 MB Infinity Cache), launches the partition kernel
``--launches`` times round-robin over the sets, then runs a plain elementwise
copy (``torch.neg`` of a float32 tensor, out of place) of a known size. The
copy calibrates the counters: FETCH_SIZE and WRITE_SIZE are reported in KiB
per dispatch, and the copy's true traffic is its tensor size read plus the same
size written, so ``scale = true bytes / counter bytes`` for each counter.

``summarize FETCH_DIR WRITE_DIR`` reads the counter CSVs of the two passes and
writes ``profiles/traffic_<workload>.json`` with the scaled read and write
bytes per partition launch, the algorithmic KV bytes next to them, and the
digest of the kernel source the counters were taken on.

    rocprofv3 --pmc FETCH_SIZE --output-format csv -d OUT/fetch -- \\
        python3 paged-decode-lab_amd/paged_decode/traffic.py run
    rocprofv3 --pmc WRITE_SIZE --output-format csv -d OUT/write -- \\
        python3 paged-decode-lab_amd/paged_decode/traffic.py run
    python3 paged-decode-lab_amd/paged_decode/traffic.py summarize OUT/fetch OUT/write

``--private-pages`` (both steps) maps every live table entry of the workload to
a page of its own, with the same lengths and layout: the same workload without
shared pages, so a shared-prefix workload's counter bytes can be compared with
what its reads cost when nothing is shared (profiles/traffic_<workload>_private.json).
"""
import argparse
import csv
import hashlib
import json
import math
import sys
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent.parent
REPO = PACKAGE_ROOT.parent
ROTATION_BYTES = 2 << 30
COPY_BYTES = 256 << 20
SOURCES = tuple(str(p.relative_to(REPO)) for p in sorted((PACKAGE_ROOT / "paged_decode" / "csrc").glob("*.hip"))) + \
    tuple(str(p.relative_to(REPO)) for p in sorted((PACKAGE_ROOT / "paged_decode" / "csrc").glob("*.h"))) + \
    ("include/paged_decode.h",)


def source_digest():
    """Short digest of the kernel source and its header."""
    h = hashlib.sha256()
    for rel in SOURCES:
        h.update((REPO / rel).read_bytes())
    return h.hexdigest()[:16]


def partition_kernel_name(dtype_is_half, whole_rows=False):
    """Name of the partition kernel (the launch that reads K and V); a whole-row
    launch is the same kernel built to fold the states and write the output."""
    name = "partial_mfma_kernel" if dtype_is_half else "partial_kernel"
    return name + " (whole rows)" if whole_rows else name


def private_table(table, lengths, page_size, physical_pages):
    """The table with every live entry mapped to a distinct physical page (in
    entry order), entries past each sequence's end left as they are."""
    import numpy as np

    out = np.array(table, dtype=np.int32, copy=True)
    live = [(b, i) for b, n in enumerate(lengths) for i in range(-(-int(n) // page_size))]
    if len(live) > physical_pages:
        raise ValueError("more live pages than the cache holds")
    for page, (b, i) in enumerate(live):
        out[b, i] = page
    return out


def workload(args):
    from paged_decode.workload import make_workload

    w = make_workload(args.workload)
    if args.private_pages:
        w.table = private_table(w.table, w.lengths, w.layout.page_size, w.layout.physical_pages)
        w.name += "_private"
    return w


def run(args):
    import numpy as np
    import torch

    from paged_decode.runtime import DecodePlan

    w = workload(args)
    dev = torch.device("cuda", 0)
    q, k0, v0, k_scale, v_scale = w.tensors(dev)  # K/V in the workload's storage format (FP8 with scales)
    sets = max(1, math.ceil(ROTATION_BYTES / (2 * k0.numel() * k0.element_size())))
    ks = [k0] + [k0.clone() for _ in range(sets - 1)]
    vs = [v0] + [v0.clone() for _ in range(sets - 1)]
    plan = DecodePlan(w.layout, w.table, w.lengths, device=dev, split_tokens=w.split_tokens)
    # A call that is one whole-row launch is measured as such (it is the call's only kernel).
    stage = plan.run if plan.launches(q.dtype, k0.dtype) == 1 else plan.run_partial
    print(f"[traffic] {w.name}: {args.launches} partition launches over {sets} K/V sets", flush=True)
    for i in range(args.launches):
        stage(q, ks[i % sets], vs[i % sets], k_scale=k_scale, v_scale=v_scale)
    torch.cuda.synchronize()
    src = torch.randn(COPY_BYTES // 4, device=dev)
    dst = torch.empty_like(src)
    for _ in range(args.copies):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    print(f"[traffic] {args.copies} calibration copies of {COPY_BYTES} bytes", flush=True)


def read_counter(directory, counter):
    """{kernel name: [values per dispatch]} for one counter from rocprofv3 CSVs."""
    per_kernel = {}
    files = sorted(Path(directory).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {directory}")
    for path in files:
        with open(path, newline="") as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") != counter:
                    continue
                per_kernel.setdefault(row["Kernel_Name"], []).append(float(row["Counter_Value"]))
    return per_kernel


def pick(per_kernel, needle):
    names = [n for n in per_kernel if needle in n and "merge" not in n]
    if len(names) != 1:
        raise SystemExit(f"expected one kernel matching {needle!r}, found {names}")
    values = per_kernel[names[0]]
    return names[0], values


def summarize(args):
    from paged_decode.metrics import kv_bytes, unique_token_bytes
    import numpy as np

    w = workload(args)
    L = w.layout
    logical = kv_bytes(w.lengths, L.kv_heads, L.head_dim, w.element_size)
    unique = unique_token_bytes(w.table, w.lengths, L.page_size, L.kv_heads, L.head_dim, w.element_size)
    kernel = partition_kernel_name(w.dtype == np.float16 or not w.native)
    record = {"workload": w.name, "kernel": kernel, "algorithmic_bytes_per_launch": logical,
              "unique_page_bytes_per_launch": unique}
    total = 0.0
    for counter, directory, key in (("FETCH_SIZE", args.fetch_dir, "read"), ("WRITE_SIZE", args.write_dir, "write")):
        per_kernel = read_counter(directory, counter)
        # rocprofv3 prints the symbol mangled when it cannot demangle the
        # _Float16 / __bf16 template arguments: match the kernel's own name.
        name, values = pick(per_kernel, kernel)
        _, copies = pick(per_kernel, "neg_kernel")
        copy_kib = sum(copies) / len(copies)
        scale = COPY_BYTES / (copy_kib * 1024.0)
        kib = sum(values) / len(values)
        scaled = kib * 1024.0 * scale
        total += scaled
        record[f"{counter.lower()}_kib_per_launch"] = round(kib, 1)
        record[f"{counter.lower()}_copy_kib"] = round(copy_kib, 1)
        record[f"{counter.lower()}_scale"] = round(scale, 4)
        record[f"hbm_{key}_bytes_per_launch"] = round(scaled)
        record[f"{counter.lower()}_launches"] = len(values)
        record["kernel_symbol"] = name
    record["hbm_bytes_per_launch"] = round(total)
    record["traffic_over_algorithmic"] = round(total / logical, 4)
    record["traffic_over_unique_pages"] = round(total / unique, 4)
    record["copy_bytes"] = COPY_BYTES
    record["source_digest"] = source_digest()
    flag = " --private-pages" if args.private_pages else ""
    record["commands"] = [
        "rocprofv3 --pmc FETCH_SIZE --output-format csv -d gpurun_out/pmc_fetch -- "
        f"python3 paged-decode-lab_amd/paged_decode/traffic.py run --workload {args.workload}{flag}",
        "rocprofv3 --pmc WRITE_SIZE --output-format csv -d gpurun_out/pmc_write -- "
        f"python3 paged-decode-lab_amd/paged_decode/traffic.py run --workload {args.workload}{flag}",
        f"python3 paged-decode-lab_amd/paged_decode/traffic.py summarize gpurun_out/pmc_fetch gpurun_out/pmc_write "
        f"--workload {args.workload}{flag}",
    ]
    out = REPO / "profiles" / f"traffic_{w.name}.json"
    out.parent.mkdir(exist_ok=True)
    out.write_text(json.dumps(record, indent=2) + "\n")
    print(json.dumps(record, indent=2))


def main(argv=None):
    # Run as a script, this file's directory leads sys.path; the package root must instead.
    here = str(Path(__file__).resolve().parent)
    sys.path[:] = [x for x in sys.path if Path(x or ".").resolve() != Path(here)]
    sys.path.insert(0, str(PACKAGE_ROOT))
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = p.add_subparsers(dest="cmd", required=True)
    r = sub.add_parser("run")
    r.add_argument("--workload", default="llama3_8b_b4_l4096")
    r.add_argument("--launches", type=int, default=24)
    r.add_argument("--copies", type=int, default=4)
    r.add_argument("--private-pages", action="store_true")
    s = sub.add_parser("summarize")
    s.add_argument("fetch_dir")
    s.add_argument("write_dir")
    s.add_argument("--workload", default="llama3_8b_b4_l4096")
    s.add_argument("--private-pages", action="store_true")
    args = p.parse_args(argv)
    return run(args) if args.cmd == "run" else summarize(args)


if __name__ == "__main__":
    sys.exit(main())
