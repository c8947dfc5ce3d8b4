"""Expert-dispatch telemetry over libqmoe's C ABI (qmoe_residency_*).

MoEResidencyTracker and MoEMetrics mirror the reference's host bookkeeping
(src/layers/moe_residency.h:35-69, src/telemetry/metrics.h:15-17): per-expert
dispatch frequencies, the resident set (the resident_k most dispatched experts,
frequency > 0, descending frequency) and the cold counter (dispatches to an
expert that was not resident at dispatch time).  Errors raise RuntimeError
(QmoeError) with the reference's messages.

Feeds from the layer:
  record_dispatches(topk_idx)  the forward's routing ids in token-major order:
                               exactly the reference's per-dispatch semantics;
  record_counts(histogram)     the device histogram that MoELayer.set_expert_counts
                               accumulates (one batch: cold by the resident set at
                               the batch's start; no host copy of the ids).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from ._lib import QmoeMoeMetrics, check, lib


@dataclass
class MoEMetrics:
    cold_dispatch_count: int = 0


class MoEResidencyTracker:
    def __init__(self, n_experts: int, resident_k: int):
        h = ctypes.c_void_p()
        check(lib().qmoe_residency_create(int(n_experts), int(resident_k), ctypes.byref(h)))
        self._handle = h
        self.n_experts = int(n_experts)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            lib().qmoe_residency_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def record_dispatch(self, expert_id: int) -> None:
        ids = (ctypes.c_int32 * 1)(int(expert_id))
        check(lib().qmoe_residency_record(self._handle, ids, 1))

    def record_dispatches(self, expert_ids) -> None:
        """record_dispatch for each id in order (a tensor is copied to the host)."""
        if hasattr(expert_ids, "detach"):
            expert_ids = expert_ids.detach().cpu().numpy()
        a = np.ascontiguousarray(np.asarray(expert_ids).reshape(-1), dtype=np.int32)
        check(lib().qmoe_residency_record(self._handle, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                          int(a.size)))

    def record_counts(self, counts) -> None:
        """One batch from a per-expert histogram of n_experts counts."""
        if hasattr(counts, "detach"):
            counts = counts.detach().cpu().numpy()
        c = np.asarray(counts)
        if c.ndim != 1 or (c.size and c.min() < 0):
            raise ValueError(f"counts expected a 1-d array of non-negative counts, got shape {c.shape}")
        a = np.ascontiguousarray(c, dtype=np.uint64)
        check(lib().qmoe_residency_record_counts(self._handle, a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                                                 int(a.size)))

    def is_resident(self, expert_id: int) -> bool:
        return bool(lib().qmoe_residency_is_resident(self._handle, int(expert_id)))

    def cold_dispatch_count(self) -> int:
        return self.snapshot_metrics().cold_dispatch_count

    def snapshot_metrics(self) -> MoEMetrics:
        m = QmoeMoeMetrics()
        check(lib().qmoe_residency_metrics(self._handle, ctypes.byref(m)))
        return MoEMetrics(int(m.cold_dispatch_count))

    def resident_set(self) -> list:
        out = (ctypes.c_int32 * self.n_experts)()
        n = lib().qmoe_residency_resident_set(self._handle, out, self.n_experts)
        return [int(out[i]) for i in range(n)]

    def frequencies(self) -> list:
        out = (ctypes.c_uint64 * self.n_experts)()
        check(lib().qmoe_residency_frequencies(self._handle, out, self.n_experts))
        return [int(v) for v in out]

    def reset(self) -> None:
        lib().qmoe_residency_reset(self._handle)
