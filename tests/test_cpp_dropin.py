"""Runs tests/cpp/test_moe_layer (the reference's test_moe.cpp cases through the
C++ drop-in include/qmoe_layer.hpp).  Host-only cases on the CPU; all on GPU."""
import os
import subprocess

import pytest

from qwenium_amd import build as qbuild


def binary():
    if not os.path.exists(qbuild.CPP_TEST_BIN):
        qbuild.build_cpp_tests()
    return qbuild.CPP_TEST_BIN


def test_cpp_dropin_host_only():
    res = subprocess.run([binary(), "--host-only"], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "19 tests, 0 failures" in res.stdout


@pytest.mark.gpu
def test_cpp_dropin_gpu(gpu):
    res = subprocess.run([binary()], capture_output=True, text=True, timeout=120)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "28 tests, 0 failures" in res.stdout
