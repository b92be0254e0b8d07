"""Runs the C++ programs of tests/cpp/, which use the public C++17 API
(include/cuvs/neighbors/*.hpp) the way the reference's callers do.

- test_api_cpu (no GPU): CGRA v1 files written by the reference's own
  save_index load with the right fields and save back byte for byte; load
  errors; argument validation; the dispatch counter API.
- test_api_gpu (GPU): the FAISS v1.8 adapter flow and known answers, the
  dispatch test with its exact answers, the exact route and the brute_force
  namespace, build -> save -> load -> search recall.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "bin")


def run(name, *args):
    exe = os.path.join(BIN, name)
    if not os.path.exists(exe):
        pytest.fail(f"{exe} is missing: build with `make -C tests/cpp` (or __graft_entry__.build())")
    p = subprocess.run([exe, *args], capture_output=True, text=True, timeout=600)
    print(p.stdout)
    print(p.stderr)
    assert p.returncode == 0, p.stderr


def test_api_cpu(tmp_path):
    run("test_api_cpu", os.path.join(HERE, "golden"), str(tmp_path))


@pytest.mark.gpu
def test_api_gpu(tmp_path):
    run("test_api_gpu", str(tmp_path))
