"""Runs the C++ programs of tests/cpp/, which use the public C++17 API
(include/cuvs/neighbors/*.hpp) the way the reference's callers do.

- test_api_cpu (no GPU): CGRA v1 files written by the reference's own
  save_index load with the right fields and save back byte for byte; load
  errors; argument validation; the dispatch counter API.
- test_api_gpu (GPU): the FAISS v1.8 adapter flow and known answers, the
  dispatch test with its exact answers, the exact route and the brute_force
  namespace, build -> save -> load -> search recall.
- test_loaders (no GPU): fvecs/ivecs and Cohere .bin readers.
- asan_test_api_cpu, asan_test_loaders (no GPU): the two above with the
  library's host sources compiled in under AddressSanitizer (leaks
  included) and UndefinedBehaviorSanitizer.
- cohere_wiki_validation (GPU): the reference's end-to-end harness CLI on
  synthetic Cohere-format files, exact route and graph route, with the index
  saved by one run and loaded by the next.
"""
import os
import re
import struct
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "bin")


def run(name, *args, env=None):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is missing: build with `make -C tests/cpp` (or __graft_entry__.build())")
    p = subprocess.run([exe, *args], capture_output=True, text=True, timeout=600,
                       env=None if env is None else {**os.environ, **env})
    print(p.stdout)
    print(p.stderr)
    assert p.returncode == 0, p.stderr
    return p.stdout


def test_api_cpu(tmp_path):
    run("test_api_cpu", os.path.join(HERE, "golden"), str(tmp_path))


@pytest.mark.gpu
def test_api_gpu(tmp_path):
    run("test_api_gpu", str(tmp_path))


def test_loaders(tmp_path):
    run("test_loaders", str(tmp_path))


SANITIZE = {"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


def test_host_code_under_sanitizers(tmp_path):
    for sub in ("api", "loaders"):
        (tmp_path / sub).mkdir()
    run("asan_test_api_cpu", os.path.join(HERE, "golden"), str(tmp_path / "api"), env=SANITIZE)
    run("asan_test_loaders", str(tmp_path / "loaders"), env=SANITIZE)


def write_bin(path, a):
    """Cohere .bin: int32 rows, int32 cols, row-major payload
    (scripts/download_cohere_wiki.py:57-71)."""
    with open(path, "wb") as f:
        f.write(struct.pack("<ii", *a.shape))
        a.tofile(f)


@pytest.mark.gpu
def test_cohere_harness(tmp_path, cvs):
    import oracle

    n, d, q, k = 12000, 1024, 100, 10
    base = cvs.synth_clustered(777, cvs.STREAM_BASE, n, d)
    queries = cvs.synth_clustered(777, cvs.STREAM_QUERIES, q, d)
    gt, _ = oracle.bf_fp64(base, queries, k, threads=8)
    paths = [str(tmp_path / f) for f in ("base.bin", "queries.bin", "gt.bin")]
    write_bin(paths[0], base)
    write_bin(paths[1], queries)
    write_bin(paths[2], gt.astype(np.int32))

    def recalls(out):
        return [float(x) for x in re.findall(r"recall@10 = ([0-9.]+)", out)]

    exact = run("cohere_wiki_validation", *paths, "10", "1", "2", "0")
    assert "PASS" in exact and recalls(exact)[0] >= 0.99
    idx = str(tmp_path / "index.cgra")
    graph = run("cohere_wiki_validation", *paths, "10", "1", "2", "64", idx)
    assert "PASS" in graph and os.path.getsize(idx) > 0
    loaded = run("cohere_wiki_validation", *paths, "10", "1", "2", "64", "", idx)
    assert "Load time" in loaded and "PASS" in loaded
    # The loaded index searches exactly as the one it was saved from.
    assert recalls(loaded)[0] == recalls(graph)[0]


# ---- the reference's own caller programs, compiled unchanged -----------------
# tests/cpp/Makefile compiles the reference's tests/test_metal_search.cpp,
# tests/test_cohere_wiki_validation.cpp, tests/test_l2_distance.cpp and
# tests/test_sift_loader.cpp from the reference tree against include/ and
# links them to libcuvs_silicon (where the reference sources are present; the
# binaries then travel with the tree).

REFERENCE_TESTS = os.environ.get("CVS_REFERENCE_DIR", "/root/reference") + "/tests"
REF_PROGRAMS = ("ref_test_metal_search", "ref_test_cohere_wiki_validation", "ref_test_l2_distance",
                "ref_test_sift_loader")


def ref_program(name):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        if os.path.isdir(REFERENCE_TESTS):
            pytest.fail(f"{exe} was not built although the reference sources are present")
        pytest.skip(f"{name} is built only where the reference sources are present")
    return name


def test_reference_callers_compile_unchanged():
    """Where the reference is present, every caller program was built."""
    if not os.path.isdir(REFERENCE_TESTS):
        pytest.skip("reference sources not present")
    for name in REF_PROGRAMS:
        assert os.path.exists(os.path.join(BIN, name)), name


def test_reference_l2_distance_program():
    """The reference's known answers for squared_l2_distance_128
    (tests/test_l2_distance.cpp:19-49) against this library's function."""
    run(ref_program("ref_test_l2_distance"))


def test_reference_sift_loader_program(tmp_path):
    """The reference's loader tests (tests/test_sift_loader.cpp) against
    this library's fvecs/ivecs readers; it writes its fixtures to the
    working directory's temp paths."""
    exe = os.path.join(BIN, ref_program("ref_test_sift_loader"))
    p = subprocess.run([exe], capture_output=True, text=True, timeout=600, cwd=str(tmp_path))
    print(p.stdout, p.stderr)
    assert p.returncode == 0, p.stderr


@pytest.mark.gpu
def test_reference_metal_search_program():
    """tests/test_metal_search.cpp: cagra::build + search must launch GPU
    kernels (metal_dispatch_count() > 0 after the search)."""
    run(ref_program("ref_test_metal_search"))


@pytest.mark.gpu
def test_reference_cohere_harness_program(tmp_path, cvs):
    """The reference's validation harness (tests/test_cohere_wiki_validation
    .cpp), unchanged, on synthetic Cohere-format files: the exact route
    (graph_degree 0) and the graph route with save and load.  The harness
    asserts its own recall bar."""
    import oracle

    name = ref_program("ref_test_cohere_wiki_validation")
    n, d, q, k = 12000, 1024, 100, 10
    base = cvs.synth_clustered(778, cvs.STREAM_BASE, n, d)
    queries = cvs.synth_clustered(778, cvs.STREAM_QUERIES, q, d)
    gt, _ = oracle.bf_fp64(base, queries, k, threads=8)
    paths = [str(tmp_path / f) for f in ("base.bin", "queries.bin", "gt.bin")]
    write_bin(paths[0], base)
    write_bin(paths[1], queries)
    write_bin(paths[2], gt.astype(np.int32))
    exact = run(name, *paths, "10", "1", "2", "0")
    assert "recall@10" in exact
    idx = str(tmp_path / "index.cgra")
    run(name, *paths, "10", "1", "2", "64", idx)
    assert os.path.getsize(idx) > 0
    run(name, *paths, "10", "1", "2", "64", "", idx)
