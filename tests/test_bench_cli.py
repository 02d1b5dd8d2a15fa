"""bench.py's command-line contract, on the CPU (no GPU work is started)."""
import subprocess

import pytest
import sys
from pathlib import Path

from gpu_util import no_child_processes_after_gpu_init

REPO = Path(__file__).resolve().parent.parent


def run_bench(*args):
    no_child_processes_after_gpu_init()
    return subprocess.run([sys.executable, str(REPO / "bench.py"), *args], capture_output=True, text=True,
                          timeout=120)


def test_more_than_one_gpu_is_refused_with_a_message():
    result = run_bench("--gpus", "2")
    assert result.returncode == 2
    assert "one GPU" in result.stderr and result.stdout == ""


def test_existing_output_file_is_never_overwritten(tmp_path):
    report = tmp_path / "report.json"
    report.write_text("keep me")
    result = run_bench("--output", str(report))
    assert result.returncode == 2
    assert "never overwrites" in result.stderr
    assert report.read_text() == "keep me"


def test_invalid_step_counts_are_refused():
    assert run_bench("--steps", "0").returncode == 2
    assert run_bench("--warmup", "-1").returncode == 2


def load_bench():
    import importlib.util

    spec = importlib.util.spec_from_file_location("bench_under_test", REPO / "bench.py")
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


def test_revision_without_git_metadata_reports_the_build_record(monkeypatch, tmp_path):
    """A copy of the tree without .git (as shipped to a GPU host) reports the
    commit and dirty flag the native libraries were built from."""
    bench = load_bench()
    from paged_decode import _build

    record = tmp_path / "_build_info.json"
    monkeypatch.setattr(_build, "BUILD_INFO", record)
    monkeypatch.setattr(_build, "git_head", lambda repo=None: None)
    assert bench.revision()["sha"] is None  # no record yet
    record.write_text('{"sha": "0123abcd", "dirty": false, "source_digest": "%s", "built_utc": "t"}'
                      % _build.source_digest())
    rev = bench.revision()
    assert rev["sha"] == "0123abcd" and rev["dirty"] is False and rev["build_sources_match_tree"] is True
    record.write_text('{"sha": "0123abcd", "dirty": true, "source_digest": "stale", "built_utc": "t"}')
    rev = bench.revision()
    assert rev["dirty"] is True and rev["build_sources_match_tree"] is False


def test_build_record_names_this_checkout(monkeypatch, tmp_path):
    """The record a build writes: this checkout's HEAD (None without git metadata) and the sources' digest."""
    from paged_decode import _build

    monkeypatch.setattr(_build, "BUILD_INFO", tmp_path / "_build_info.json")
    info = _build.write_build_info()
    assert _build.build_info() == info
    assert info["sha"] == _build.git_head() and info["source_digest"] == _build.source_digest()
    if info["sha"] is not None:
        assert len(info["sha"]) == 40 and info["dirty"] in (True, False, None)


def test_sweep_shapes_are_well_formed():
    """Every named sweep shape builds valid metadata: lengths within the
    table, page ids in range, the reserve and the shared prefix respected."""
    from paged_decode import sweep
    from paged_decode.layout import validate_metadata

    listed = sweep.shapes(["all"])
    assert {name for name, _ in listed} == set(sweep.SWEEPS)
    assert len({shape for _, shape in listed}) == len(listed)
    for _, shape in listed:
        layout, table, lengths, max_context = sweep.metadata(shape)
        validate_metadata(layout, table, lengths)
        assert max_context <= table.shape[1] * layout.page_size
        assert int(lengths.max()) * shape.reserve <= table.shape[1] * layout.page_size
        if shape.shared_prefix:
            shared = int(-(-int(lengths.max()) // layout.page_size) * shape.shared_prefix)
            live = lengths >= shared * layout.page_size
            assert (table[live, :shared] == table[live][0, :shared]).all()
    with pytest.raises(ValueError):
        sweep.shapes(["nonesuch"])
