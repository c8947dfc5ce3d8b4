"""Host-side sanitizer run (AddressSanitizer + UndefinedBehaviorSanitizer).

    python -m qwenium_amd.sanitize [pytest -k expression]

Builds libqmoe.so and the C++ drop-in test with host-instrumented code
(qwenium_amd.build.build_sanitized: every -fsanitize= after -Xarch_host, the
gfx950 device code as usual), then runs, with the sanitizer runtime preloaded
into the Python interpreter:
  - tests/cpp test binary --host-only (constructor contract, GGUF through the
    C++ wrapper, the residency tracker): no GPU needed;
  - pytest -m "not gpu" over the library's host code (ABI validation, GGUF
    reader, residency tracker), loading the sanitized library (QMOE_LIB).
Exits non-zero on any sanitizer report or test failure.  CPU only.
"""
from __future__ import annotations

import os
import subprocess
import sys

from . import build as B

DEFAULT_K = "test_abi or test_gguf or test_residency"


def _runtime() -> str:
    out = subprocess.run([B._hipcc(), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                         text=True).stdout.strip()
    if not out or not os.path.exists(out):
        raise SystemExit("no libclang_rt.asan-x86_64.so next to hipcc")
    return out


def main(argv=None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    kexpr = argv[0] if argv else DEFAULT_K
    B.build_sanitized()
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1:detect_odr_violation=0"
    env["UBSAN_OPTIONS"] = "print_stacktrace=1:halt_on_error=1"
    rt = _runtime()
    env["LD_LIBRARY_PATH"] = os.path.dirname(rt) + (":" + env["LD_LIBRARY_PATH"] if env.get("LD_LIBRARY_PATH") else "")
    print("[sanitize] C++ host-only cases", flush=True)
    rc = subprocess.run([B.SAN_TEST_BIN, "--host-only"], env=env).returncode
    if rc:
        return rc
    env["LD_PRELOAD"] = rt
    env["QMOE_LIB"] = B.SAN_LIB
    print(f"[sanitize] pytest -m 'not gpu' -k '{kexpr}'", flush=True)
    return subprocess.run([sys.executable, "-m", "pytest", os.path.join(B.REPO_DIR, "tests"), "-q", "-m", "not gpu",
                           "-k", kexpr, "-p", "no:cacheprovider"], env=env).returncode


if __name__ == "__main__":
    sys.exit(main())
