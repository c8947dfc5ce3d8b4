"""ctypes binding of libqmoe.so (the C ABI declared in include/qmoe.h).

The shared library is built in-tree by qwenium_amd.build.build().  Loading
fails loudly when it is missing: there is no CPU fallback for the layer.
"""
from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
# QMOE_LIB: another build of the same library (the host-sanitizer build,
# qwenium_amd.sanitize); default: the in-tree libqmoe.so
LIB_PATH = os.environ.get("QMOE_LIB") or os.path.join(PKG_DIR, "libqmoe.so")

TYPE_F32 = 0
TYPE_Q4_0 = 2
TYPE_Q8_0 = 8

QMOE_OK = 0
QMOE_ERR_NULL = 1
QMOE_ERR_SHAPE = 2
QMOE_ERR_TYPE = 3
QMOE_ERR_VALUE = 4
QMOE_ERR_CAPACITY = 5
QMOE_ERR_HIP = 6
QMOE_ERR_SYNC = 7

# every function declared in include/qmoe.h
EXPORTED = (
    "qmoe_last_error",
    "qmoe_layer_create",
    "qmoe_layer_destroy",
    "qmoe_layer_n_embd",
    "qmoe_layer_build_prefill_copies",
    "qmoe_workspace_create",
    "qmoe_workspace_destroy",
    "qmoe_workspace_capacity",
    "qmoe_workspace_check",
    "qmoe_layer_forward",
    "qmoe_layer_forward_norm",
    "qmoe_layer_forward_norm_chain",
    "qmoe_layer_forward_static",
    "qmoe_layer_set_phase_events",
    "qmoe_rms_norm",
    "qmoe_rms_partials",
    "qmoe_synth_f32",
    "qmoe_synth_quant",
    "qmoe_gguf_open",
    "qmoe_gguf_close",
    "qmoe_gguf_info",
    "qmoe_gguf_get_u32",
    "qmoe_gguf_get_f32",
    "qmoe_gguf_get_str",
    "qmoe_gguf_tensor_name",
    "qmoe_gguf_find",
    "qmoe_gguf_read",
    "qmoe_gguf_upload",
    "qmoe_gguf_tensor_view",
    "qmoe_layer_set_expert_counts",
    "qmoe_geglu_layer_create",
    "qmoe_layer_forward_routed",
    "qmoe_layer_forward_gemma4",
    "qmoe_gemma4_moe_inputs",
    "qmoe_gelu_f16_table",
    "qmoe_residency_create",
    "qmoe_residency_destroy",
    "qmoe_residency_record",
    "qmoe_residency_record_counts",
    "qmoe_residency_is_resident",
    "qmoe_residency_metrics",
    "qmoe_residency_resident_set",
    "qmoe_residency_frequencies",
    "qmoe_residency_reset",
)


class QmoeTensor(ctypes.Structure):
    _fields_ = [
        ("data", ctypes.c_void_p),
        ("type", ctypes.c_int32),
        ("n_dims", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("nb", ctypes.c_uint64 * 4),
    ]


class QmoeHparams(ctypes.Structure):
    _fields_ = [
        ("n_experts", ctypes.c_int32),
        ("top_k", ctypes.c_int32),
        ("ffn_dim", ctypes.c_int32),
        ("has_shared_expert", ctypes.c_int32),
    ]


class QmoeDebug(ctypes.Structure):
    _fields_ = [
        ("logits", ctypes.c_void_p),
        ("topk_idx", ctypes.c_void_p),
        ("topk_w", ctypes.c_void_p),
        ("sh_gate", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
        ("rows", ctypes.c_void_p),
        ("router_approx", ctypes.c_void_p),
        ("router_bound", ctypes.c_void_p),
        ("h_qs", ctypes.c_void_p),
        ("h_d", ctypes.c_void_p),
        ("h_fixed", ctypes.c_void_p),
        ("exp_down", ctypes.c_void_p),
    ]


class QmoeGgufTensor(ctypes.Structure):
    _fields_ = [
        ("type", ctypes.c_int32),
        ("n_dims", ctypes.c_int32),
        ("ne", ctypes.c_int64 * 4),
        ("file_offset", ctypes.c_uint64),
        ("nbytes", ctypes.c_uint64),
    ]


class QmoeMoeMetrics(ctypes.Structure):
    _fields_ = [("cold_dispatch_count", ctypes.c_uint64)]


class QmoeError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(message)
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Loads libqmoe.so once; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER
    vp = ctypes.c_void_p
    L.qmoe_last_error.restype = ctypes.c_char_p
    L.qmoe_last_error.argtypes = []
    L.qmoe_layer_create.restype = ctypes.c_int
    L.qmoe_layer_create.argtypes = [P(QmoeTensor)] * 8 + [P(QmoeHparams), P(vp)]
    L.qmoe_layer_destroy.restype = ctypes.c_int
    L.qmoe_layer_destroy.argtypes = [vp]
    L.qmoe_layer_n_embd.restype = ctypes.c_int
    L.qmoe_layer_n_embd.argtypes = [vp]
    L.qmoe_layer_build_prefill_copies.restype = ctypes.c_int
    L.qmoe_layer_build_prefill_copies.argtypes = [vp]
    L.qmoe_workspace_create.restype = ctypes.c_int
    L.qmoe_workspace_create.argtypes = [vp, ctypes.c_int32, P(vp)]
    L.qmoe_workspace_destroy.restype = ctypes.c_int
    L.qmoe_workspace_destroy.argtypes = [vp]
    L.qmoe_workspace_capacity.restype = ctypes.c_int32
    L.qmoe_workspace_capacity.argtypes = [vp]
    L.qmoe_workspace_check.restype = ctypes.c_int
    L.qmoe_workspace_check.argtypes = [vp, ctypes.POINTER(ctypes.c_int32)]
    L.qmoe_layer_forward.restype = ctypes.c_int
    L.qmoe_layer_forward.argtypes = [vp, vp, vp, ctypes.c_int32, vp, vp, P(QmoeDebug), vp]
    L.qmoe_layer_forward_static.restype = ctypes.c_int
    L.qmoe_layer_forward_static.argtypes = [vp, vp, ctypes.c_int32, vp, vp, vp]
    L.qmoe_layer_forward_norm.restype = ctypes.c_int
    L.qmoe_layer_forward_norm.argtypes = [vp, vp, vp, vp, ctypes.c_float, ctypes.c_int32, vp, P(QmoeDebug), vp]
    L.qmoe_layer_set_phase_events.restype = ctypes.c_int
    L.qmoe_layer_set_phase_events.argtypes = [vp, P(vp)]
    L.qmoe_rms_norm.restype = ctypes.c_int
    L.qmoe_rms_norm.argtypes = [vp, vp, ctypes.c_int32, ctypes.c_int32, ctypes.c_float, vp, vp]
    L.qmoe_rms_partials.restype = ctypes.c_int
    L.qmoe_rms_partials.argtypes = [vp, ctypes.c_int32, ctypes.c_int32, vp, vp]
    L.qmoe_layer_forward_norm_chain.restype = ctypes.c_int
    L.qmoe_layer_forward_norm_chain.argtypes = [vp, vp, vp, vp, vp, ctypes.c_float, ctypes.c_int32, vp, vp,
                                                P(QmoeDebug), vp]
    L.qmoe_synth_f32.restype = ctypes.c_int
    L.qmoe_synth_f32.argtypes = [vp, ctypes.c_int64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_double,
                                 ctypes.c_double, vp]
    L.qmoe_synth_quant.restype = ctypes.c_int
    L.qmoe_synth_quant.argtypes = [vp, ctypes.c_int32, ctypes.c_int64, ctypes.c_int64, ctypes.c_uint64,
                                   ctypes.c_uint64, ctypes.c_double, vp]
    cp = ctypes.c_char_p
    L.qmoe_gguf_open.restype = ctypes.c_int
    L.qmoe_gguf_open.argtypes = [cp, P(vp)]
    L.qmoe_gguf_close.restype = None
    L.qmoe_gguf_close.argtypes = [vp]
    L.qmoe_gguf_info.restype = ctypes.c_int
    L.qmoe_gguf_info.argtypes = [vp, P(ctypes.c_uint32), P(ctypes.c_int64), P(ctypes.c_int64), P(ctypes.c_uint64)]
    L.qmoe_gguf_get_u32.restype = ctypes.c_int
    L.qmoe_gguf_get_u32.argtypes = [vp, cp, P(ctypes.c_uint32)]
    L.qmoe_gguf_get_f32.restype = ctypes.c_int
    L.qmoe_gguf_get_f32.argtypes = [vp, cp, P(ctypes.c_float)]
    L.qmoe_gguf_get_str.restype = ctypes.c_int
    L.qmoe_gguf_get_str.argtypes = [vp, cp, P(cp)]
    L.qmoe_gguf_tensor_name.restype = ctypes.c_int
    L.qmoe_gguf_tensor_name.argtypes = [vp, ctypes.c_int64, P(cp)]
    L.qmoe_gguf_find.restype = ctypes.c_int
    L.qmoe_gguf_find.argtypes = [vp, cp, P(QmoeGgufTensor)]
    L.qmoe_gguf_read.restype = ctypes.c_int
    L.qmoe_gguf_read.argtypes = [vp, cp, vp, ctypes.c_uint64]
    L.qmoe_gguf_upload.restype = ctypes.c_int
    L.qmoe_gguf_upload.argtypes = [vp, cp, vp, ctypes.c_uint64, vp]
    L.qmoe_gguf_tensor_view.restype = ctypes.c_int
    L.qmoe_gguf_tensor_view.argtypes = [P(QmoeGgufTensor), vp, P(QmoeTensor)]
    L.qmoe_geglu_layer_create.restype = ctypes.c_int
    L.qmoe_geglu_layer_create.argtypes = [P(QmoeTensor)] * 3 + [P(QmoeHparams), P(vp)]
    L.qmoe_layer_forward_routed.restype = ctypes.c_int
    L.qmoe_layer_forward_routed.argtypes = [vp, vp, vp, vp, ctypes.c_int32, vp, P(QmoeDebug), vp]
    L.qmoe_layer_forward_gemma4.restype = ctypes.c_int
    L.qmoe_layer_forward_gemma4.argtypes = [vp, vp, vp, vp, vp, ctypes.c_float, ctypes.c_int32, vp, P(QmoeDebug), vp]
    L.qmoe_gemma4_moe_inputs.restype = ctypes.c_int
    L.qmoe_gemma4_moe_inputs.argtypes = [vp, vp, vp, ctypes.c_float, ctypes.c_int32, ctypes.c_int32, vp, vp, vp]
    L.qmoe_gelu_f16_table.restype = ctypes.c_int
    L.qmoe_gelu_f16_table.argtypes = [P(ctypes.c_uint16)]
    L.qmoe_layer_set_expert_counts.restype = ctypes.c_int
    L.qmoe_layer_set_expert_counts.argtypes = [vp, vp]
    L.qmoe_residency_create.restype = ctypes.c_int
    L.qmoe_residency_create.argtypes = [ctypes.c_int32, ctypes.c_int32, P(vp)]
    L.qmoe_residency_destroy.restype = None
    L.qmoe_residency_destroy.argtypes = [vp]
    L.qmoe_residency_record.restype = ctypes.c_int
    L.qmoe_residency_record.argtypes = [vp, P(ctypes.c_int32), ctypes.c_int64]
    L.qmoe_residency_record_counts.restype = ctypes.c_int
    L.qmoe_residency_record_counts.argtypes = [vp, P(ctypes.c_uint64), ctypes.c_int32]
    L.qmoe_residency_is_resident.restype = ctypes.c_int
    L.qmoe_residency_is_resident.argtypes = [vp, ctypes.c_int32]
    L.qmoe_residency_metrics.restype = ctypes.c_int
    L.qmoe_residency_metrics.argtypes = [vp, P(QmoeMoeMetrics)]
    L.qmoe_residency_resident_set.restype = ctypes.c_int32
    L.qmoe_residency_resident_set.argtypes = [vp, P(ctypes.c_int32), ctypes.c_int32]
    L.qmoe_residency_frequencies.restype = ctypes.c_int
    L.qmoe_residency_frequencies.argtypes = [vp, P(ctypes.c_uint64), ctypes.c_int32]
    L.qmoe_residency_reset.restype = None
    L.qmoe_residency_reset.argtypes = [vp]
    _lib = L
    return L


def last_error() -> str:
    return lib().qmoe_last_error().decode()


def check(rc: int) -> None:
    if rc != QMOE_OK:
        raise QmoeError(rc, last_error())


def block_bytes(type_id: int) -> int:
    return {TYPE_Q4_0: 18, TYPE_Q8_0: 34, TYPE_F32: 4}[type_id]


def row_bytes(type_id: int, n: int) -> int:
    if type_id == TYPE_F32:
        return 4 * n
    return (n // 32) * block_bytes(type_id)


def make_tensor(ptr: int, type_id: int, ne: tuple, nb: tuple | None = None) -> QmoeTensor:
    """A ggml-style view: ne[0] contiguous; nb defaults to the contiguous strides."""
    t = QmoeTensor()
    t.data = ptr
    t.type = type_id
    t.n_dims = len(ne)
    if nb is None:
        nb = [block_bytes(type_id)]
        nb.append(row_bytes(type_id, ne[0]))
        for i in range(2, len(ne)):
            nb.append(nb[-1] * ne[i - 1])
    for i in range(4):
        t.ne[i] = ne[i] if i < len(ne) else 1
        t.nb[i] = nb[i] if i < len(nb) else (nb[-1] * (ne[-1] if ne else 1))
    return t
