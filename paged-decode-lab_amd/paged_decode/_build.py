"""Ahead-of-time build of the native libraries, in-tree, for gfx950.

* ``libpaged_decode_hip.so`` -- HIP kernels and the C ABI of
  ``include/paged_decode.h``, compiled by ``hipcc --offload-arch=gfx950``.
* ``_C.so`` -- the thin PyTorch extension (host C++ only, compiled by the host
  compiler against torch's headers) that calls the C ABI.

Sources are compiled as written: nothing here runs torch's hipify step. Run as
``python -m paged_decode._build`` or through ``__graft_entry__.build()``.
"""
import hashlib
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
REPO = PACKAGE.parent.parent
INCLUDE = REPO / "include"
HIP_LIBRARY = PACKAGE / "libpaged_decode_hip.so"
EXTENSION = PACKAGE / "_C.so"
BUILD_INFO = PACKAGE / "_build_info.json"  # git revision and source digest of the last build
ARCH = os.environ.get("PAGED_DECODE_ARCH", "gfx950")
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

# -packed-fp32-ops keeps the device compiler from forming v_pk_{add,mul,fma}_f32.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-command-line-argument"]


def sources():
    """Every file the two libraries are compiled from."""
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp")) + sorted(CSRC.glob("*.h")) + \
        sorted(INCLUDE.glob("*.h"))


def source_digest():
    """Short digest of the native sources, compiled into ``_C`` as its build digest."""
    h = hashlib.sha256()
    for path in sources():
        h.update(path.name.encode())
        h.update(path.read_bytes())
    return h.hexdigest()[:16]


def gpu_initialised():
    """Whether this process has initialised the GPU runtime (as torch sees it)."""
    torch = sys.modules.get("torch")
    return torch is not None and torch.cuda.is_initialized()


def refuse_after_gpu_init(what):
    """Raise instead of starting a child process from a process that has
    initialised the GPU: on this stack a program started from such a process
    (a compiler, git) can take the GPU runtime down with it. Build first, in
    a process that has not touched the GPU."""
    if gpu_initialised():
        raise RuntimeError(f"{what} would start a child process from a process that has initialised the GPU; "
                           f"build the native libraries first (python -m paged_decode._build) and restart")


def _run(cmd, verbose):
    refuse_after_gpu_init(f"running {Path(str(cmd[0])).name}")
    if verbose:
        print(" ".join(str(c) for c in cmd), flush=True)
    result = subprocess.run([str(c) for c in cmd], capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(str(c) for c in cmd)}\n"
                           f"{result.stdout}\n{result.stderr}")
    noise = "is not a recognized feature for this target"
    for line in result.stderr.splitlines():
        if verbose and noise not in line:
            print(line, flush=True)


def _atomic_output(path):
    return path.with_name(path.name + f".tmp{os.getpid()}")


def build_hip_library(verbose=False, jobs=None):
    """Compile every csrc/*.hip unit for gfx950 in parallel, then link the library."""
    from concurrent.futures import ThreadPoolExecutor

    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    units = sorted(CSRC.glob("*.hip"))
    objects_dir = PACKAGE / "_build_objects"
    objects_dir.mkdir(exist_ok=True)
    compile_flags = [f for f in HIP_FLAGS if f != "-shared"]

    def compile_unit(unit):
        obj = objects_dir / (unit.stem + ".o")
        _run([hipcc, *compile_flags, "-c", "-I", INCLUDE, "-I", CSRC, "-o", obj, unit], verbose)
        return obj

    workers = jobs or max(1, min(len(units), len(os.sched_getaffinity(0)), 16))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(compile_unit, units))
    tmp = _atomic_output(HIP_LIBRARY)
    _run([hipcc, *HIP_FLAGS, "-o", tmp, *objects], verbose)
    os.replace(tmp, HIP_LIBRARY)
    shutil.rmtree(objects_dir, ignore_errors=True)
    return HIP_LIBRARY


def build_extension(verbose=False):
    import torch
    from torch.utils import cpp_extension

    cxx = os.environ.get("CXX", "g++")
    torch_lib = Path(torch.__file__).resolve().parent / "lib"
    includes = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(ROCM / "include"),
                str(INCLUDE)]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = _atomic_output(EXTENSION)
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DTORCH_API_INCLUDE_EXTENSION_H",
           "-DTORCH_EXTENSION_NAME=_C", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           f'-DPD_BUILD_DIGEST="{source_digest()}"',
           *[f"-I{p}" for p in includes],
           CSRC / "torch_ext.cpp", "-o", tmp,
           f"-L{PACKAGE}", "-lpaged_decode_hip", f"-L{torch_lib}", "-lc10", "-lc10_hip", "-ltorch",
           "-ltorch_cpu", "-ltorch_hip", "-ltorch_python", f"-L{ROCM / 'lib'}", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}", f"-Wl,-rpath,{ROCM / 'lib'}"]
    _run(cmd, verbose)
    os.replace(tmp, EXTENSION)
    return EXTENSION


def git_head(repo=REPO):
    """Commit of the repository's HEAD, read from .git's files (no git process), or None."""
    git = Path(repo) / ".git"
    try:
        head = (git / "HEAD").read_text().strip()
        if not head.startswith("ref: "):
            return head
        ref = head[5:]
        if (git / ref).exists():
            return (git / ref).read_text().strip()
        for line in (git / "packed-refs").read_text().splitlines():
            if line.endswith(" " + ref):
                return line.split()[0]
    except OSError:
        pass
    return None


def git_dirty(repo=REPO):
    """True when tracked files differ from HEAD, None when git cannot tell
    (also in a process that has initialised the GPU, which starts no git)."""
    if gpu_initialised():
        return None
    try:
        status = subprocess.check_output(["git", "status", "--porcelain", "--untracked-files=no"], cwd=repo,
                                         text=True, stderr=subprocess.DEVNULL, timeout=10)
    except (OSError, subprocess.SubprocessError):
        return None
    return bool(status.strip())


def write_build_info():
    """Record which revision and sources the libraries were built from, next to
    them (a copy of the tree without .git, e.g. on another machine, keeps it)."""
    import json
    from datetime import datetime, timezone

    sha = git_head()
    info = {"sha": sha, "dirty": git_dirty() if sha else None, "source_digest": source_digest(),
            "built_utc": datetime.now(timezone.utc).isoformat(timespec="seconds")}
    tmp = _atomic_output(BUILD_INFO)
    tmp.write_text(json.dumps(info, indent=1) + "\n")
    os.replace(tmp, BUILD_INFO)
    return info


def build_info():
    """The record write_build_info left, or None."""
    import json

    try:
        return json.loads(BUILD_INFO.read_text())
    except (OSError, ValueError):
        return None


def build(verbose=False):
    """Compile both libraries and record their revision; returns their paths."""
    paths = build_hip_library(verbose), build_extension(verbose)
    write_build_info()
    return paths


def built():
    return HIP_LIBRARY.exists() and EXTENSION.exists()


def check_loaded(extension):
    """Raise if the imported ``_C`` was built from other sources than the tree
    holds, or if the HIP library it loaded reports another ABI version than
    the header ``_C`` was compiled against: a stale build would otherwise run
    old kernels silently or reject new arguments."""
    digest = source_digest()
    if extension.build_digest() != digest:
        raise RuntimeError(f"paged_decode native build is stale (built from sources {extension.build_digest()}, "
                           f"tree holds {digest}): run `python -m paged_decode._build` and restart")
    if extension.abi_version() != extension.header_abi_version():
        raise RuntimeError(f"libpaged_decode_hip.so reports ABI {extension.abi_version()}, the extension was "
                           f"compiled for {extension.header_abi_version()}: rebuild both libraries")


if __name__ == "__main__":
    for path in build(verbose="-q" not in sys.argv):
        print(path)
