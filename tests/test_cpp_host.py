"""Runs the C++ host-mirror tests (tests/cpp/test_host.cpp): the --cpu cases here, the
--gpu cases on the GPU. The binary is built by __graft_entry__.build()."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "_build", "test_host")


def _run(flag):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} not built (run __graft_entry__.build())")
    r = subprocess.run([BIN, flag], capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr


def test_cpp_host_cpu():
    _run("--cpu")


@pytest.mark.gpu
def test_cpp_host_gpu():
    _run("--gpu")
