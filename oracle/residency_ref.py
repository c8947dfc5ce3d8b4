"""ctypes binding of oracle/_ref/libresidency_ref.so: the reference's own
MoEResidencyTracker (src/layers/moe_residency.cpp, compiled unmodified by
oracle/Makefile behind oracle/residency_ref_driver.cpp).

TEST INFRASTRUCTURE ONLY: the checker for libqmoe's qmoe_residency_* tracker.
available() is False where the library was not built (no reference tree).
"""
from __future__ import annotations

import ctypes
import os

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libresidency_ref.so")
_lib = None


def available() -> bool:
    return os.path.exists(LIB_PATH)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        L = ctypes.CDLL(LIB_PATH)
        vp, i = ctypes.c_void_p, ctypes.c_int
        L.ref_res_last_error.restype = ctypes.c_char_p
        L.ref_res_last_error.argtypes = []
        L.ref_res_create.restype = vp
        L.ref_res_create.argtypes = [i, i]
        L.ref_res_destroy.restype = None
        L.ref_res_destroy.argtypes = [vp]
        L.ref_res_record.restype = i
        L.ref_res_record.argtypes = [vp, i]
        L.ref_res_cold.restype = ctypes.c_uint64
        L.ref_res_cold.argtypes = [vp]
        L.ref_res_is_resident.restype = i
        L.ref_res_is_resident.argtypes = [vp, i]
        L.ref_res_resident_set.restype = i
        L.ref_res_resident_set.argtypes = [vp, ctypes.POINTER(i), i]
        L.ref_res_frequencies.restype = None
        L.ref_res_frequencies.argtypes = [vp, ctypes.POINTER(ctypes.c_uint64), i]
        L.ref_res_reset.restype = None
        L.ref_res_reset.argtypes = [vp]
        _lib = L
    return _lib


class RefTracker:
    """The reference tracker; methods as MoEResidencyTracker's."""

    def __init__(self, n_experts: int, resident_k: int):
        self._h = lib().ref_res_create(int(n_experts), int(resident_k))
        if not self._h:
            raise RuntimeError(lib().ref_res_last_error().decode())
        self.n_experts = int(n_experts)

    def __del__(self):
        if getattr(self, "_h", None):
            lib().ref_res_destroy(self._h)
            self._h = None

    def record_dispatch(self, expert_id: int) -> None:
        if lib().ref_res_record(self._h, int(expert_id)):
            raise RuntimeError(lib().ref_res_last_error().decode())

    def cold_dispatch_count(self) -> int:
        return int(lib().ref_res_cold(self._h))

    def is_resident(self, expert_id: int) -> bool:
        return bool(lib().ref_res_is_resident(self._h, int(expert_id)))

    def resident_set(self) -> list:
        out = (ctypes.c_int * self.n_experts)()
        n = lib().ref_res_resident_set(self._h, out, self.n_experts)
        return [int(out[i]) for i in range(n)]

    def frequencies(self) -> list:
        out = (ctypes.c_uint64 * self.n_experts)()
        lib().ref_res_frequencies(self._h, out, self.n_experts)
        return [int(v) for v in out]

    def reset(self) -> None:
        lib().ref_res_reset(self._h)
