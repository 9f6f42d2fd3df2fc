"""Runs the C++ host-layer test driver (tests/cpp/iq2_matmul_tests): the C++
counterpart of the reference's Rust API, tested like the reference's own
#[test]s (src/iq2_matmul.rs:1255-1313)."""

import os
import subprocess

import pytest

from conftest import REPO

BIN = os.path.join(REPO, "tests", "cpp", "iq2_matmul_tests")


def _run(flag):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (run __graft_entry__.build())")
    r = subprocess.run([BIN, flag], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "test result: ok" in r.stdout


def test_cpp_host_suite():
    _run("--host")


@pytest.mark.gpu
def test_cpp_gpu_suite():
    _run("--gpu")
