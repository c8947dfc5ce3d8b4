"""Host code under AddressSanitizer + UndefinedBehaviorSanitizer (no GPU).

qwenium_amd.sanitize rebuilds libqmoe.so and the C++ drop-in test with every
source's host code instrumented (the gfx950 device code as usual), runs the C++
host-only cases (constructor contract, GGUF through the C++ wrapper, residency
tracker) and the CPU tests of the ABI validation, the GGUF reader (crafted
inventories included) and the residency tracker against that library.  Any
sanitizer report aborts the run.
"""
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_host_code_under_asan_and_ubsan():
    res = subprocess.run([sys.executable, "-m", "qwenium_amd.sanitize"], cwd=REPO, capture_output=True, text=True,
                         timeout=900)
    tail = (res.stdout + res.stderr)[-3000:]
    assert res.returncode == 0, tail
    assert "19 tests, 0 failures" in res.stdout or " 0 failures" in res.stdout, tail
    assert " passed" in res.stdout and "failed" not in res.stdout, tail
