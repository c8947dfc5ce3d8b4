"""Build recipe for libqmoe.so (HIP kernels + C ABI) for gfx950.

Compiles every source under qwenium_amd/csrc with hipcc into objects under
qwenium_amd/_build and links qwenium_amd/libqmoe.so.  Always recompiles (the
driver's "does it build" check calls it on a CPU-only host; hipcc
cross-compiles gfx950 without a GPU).
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libqmoe.so")
SOURCES = [
    "route_kernels.hip",
    "expert_gemv_kernels.hip",
    "expert_f16_kernels.hip",
    "misc_kernels.hip",
    "qmoe_api.cpp",
    "gguf.cpp",
    "residency.cpp",
    "gelu_table.cpp",
]
ARCH = os.environ.get("QMOE_OFFLOAD_ARCH", "gfx950")


def _hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: install ROCm or put hipcc on PATH")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # packed FP32 VALU ops stay off (see the design notes on numerics)
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # MFMA results in VGPRs (no accumulator-register copies in the epilogues)
        "-mllvm", "-amdgpu-mfma-vgpr-form",
        "-I", os.path.join(REPO_DIR, "include"),
        "-I", CSRC,
        "-Wall",
    ]


# Host-side AddressSanitizer + UndefinedBehaviorSanitizer (each -fsanitize= after
# -Xarch_host: the host code of every source is instrumented, the gfx950 device
# code is built as usual).
SAN_DIR = os.path.join(BUILD_DIR, "san")
SAN_LIB = os.path.join(SAN_DIR, "libqmoe.so")
SAN_TEST_BIN = os.path.join(SAN_DIR, "test_moe_layer")
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-fno-omit-frame-pointer",
             "-Xarch_host", "-g"]


def _compile(src: str, verbose: bool, extra: list[str] | None = None, out_dir: str | None = None) -> str:
    obj = os.path.join(out_dir or BUILD_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [_hipcc()] + common_flags() + (extra or []) + ["-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd[1:1] = ["-x", "hip"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "is not a recognized feature for this target" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    if verbose and out.strip():
        print(out, flush=True)
    return obj


def build(verbose: bool = False, jobs: int = 5) -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp] + objs
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB_PATH)
    build_cpp_tests(verbose)
    return LIB_PATH


def build_sanitized(verbose: bool = False, jobs: int = 5) -> str:
    """The library and the C++ drop-in test with host-side ASan + UBSan, under
    qwenium_amd/_build/san (run them with qwenium_amd.sanitize)."""
    os.makedirs(SAN_DIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose, SAN_FLAGS, SAN_DIR), SOURCES))
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-shared-libsan"] + SAN_FLAGS + ["-o", SAN_LIB] + objs
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"sanitized link failed:\n{res.stdout}{res.stderr}")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-O1", "-std=c++17", "-shared-libsan"] + SAN_FLAGS + [
        "-I", os.path.join(REPO_DIR, "include"), CPP_TEST_SRC, "-o", SAN_TEST_BIN, "-L", SAN_DIR, "-lqmoe",
        "-Wl,-rpath," + SAN_DIR]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"sanitized C++ test build failed:\n{res.stdout}{res.stderr}")
    return SAN_LIB


CPP_TEST_SRC = os.path.join(REPO_DIR, "tests", "cpp", "test_moe_layer.cpp")
CPP_TEST_BIN = os.path.join(REPO_DIR, "tests", "cpp", "test_moe_layer")


def build_cpp_tests(verbose: bool = False) -> str:
    """The C++ drop-in test (tests/cpp/test_moe_layer.cpp) linked against libqmoe.so."""
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-O2", "-std=c++17", "-I", os.path.join(REPO_DIR, "include"),
           CPP_TEST_SRC, "-o", CPP_TEST_BIN, "-L", PKG_DIR, "-lqmoe",
           "-Wl,-rpath,$ORIGIN/../../qwenium_amd"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"C++ test build failed:\n{res.stdout}{res.stderr}")
    return CPP_TEST_BIN


if __name__ == "__main__":
    print(build(verbose=True))
