"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker.  The product (qwenium_amd) never
imports it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "liboracle.so")

TYPE_F32, TYPE_Q4_0, TYPE_Q8_0 = 0, 2, 8


REFERENCE_DIR = "/root/reference"


def build() -> str:
    """Compiles liboracle.so with oracle/Makefile (gcc; no GPU involved) and,
    where the reference tree is present, oracle/_ref/libresidency_ref.so from
    the reference's own MoEResidencyTracker source."""
    subprocess.run(["make", "-s", "-C", ORACLE_DIR, "-B", "CC=gcc", "liboracle.so"], check=True)
    if os.path.exists(os.path.join(REFERENCE_DIR, "src", "layers", "moe_residency.cpp")):
        subprocess.run(["make", "-s", "-C", ORACLE_DIR, "-B", "CXX=g++", f"REF={REFERENCE_DIR}",
                        "_ref/libresidency_ref.so"], check=True)
    return LIB_PATH


class QoLayer(ctypes.Structure):
    _fields_ = [
        ("n_embd", ctypes.c_int), ("n_experts", ctypes.c_int), ("top_k", ctypes.c_int),
        ("ffn_dim", ctypes.c_int), ("has_shared_expert", ctypes.c_int), ("expert_type", ctypes.c_int),
        ("w_router", ctypes.c_void_p), ("w_gate", ctypes.c_void_p), ("w_up", ctypes.c_void_p),
        ("w_down", ctypes.c_void_p), ("w_sh_gate", ctypes.c_void_p), ("w_sh_up", ctypes.c_void_p),
        ("w_sh_down", ctypes.c_void_p), ("w_sh_norm", ctypes.c_void_p),
        ("act", ctypes.c_int), ("gate_up_fused", ctypes.c_int),
    ]


class QoDebug(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("logits", "topk_idx", "topk_w", "sh_gate", "offsets", "rows", "h", "y", "sh_out", "sh_h")]


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = ctypes.CDLL(LIB_PATH)
    vp, i64, u64, f32, f64, i32 = (ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float,
                                   ctypes.c_double, ctypes.c_int)
    sig = {
        "qo_fp32_to_fp16": (ctypes.c_uint16, [f32]),
        "qo_fp16_to_fp32": (f32, [ctypes.c_uint16]),
        "qo_exp_det": (f64, [f64]),
        "qo_log_det": (f64, [f64]),
        "qo_cospi2_det": (f64, [f64]),
        "qo_hash3": (u64, [u64, u64, u64]),
        "qo_normal": (f64, [u64, u64, u64]),
        "qo_gen_normal_f32": (None, [u64, u64, f64, f64, vp, i64]),
        "qo_type_block_bytes": (ctypes.c_size_t, [i32]),
        "qo_row_bytes": (ctypes.c_size_t, [i32, i64]),
        "qo_quantize_q4_0": (None, [vp, vp, i64]),
        "qo_quantize_q8_0": (None, [vp, vp, i64]),
        "qo_quantize_q8_0_act": (None, [vp, vp, i64]),
        "qo_dequantize": (None, [i32, vp, vp, i64]),
        "qo_vec_dot": (f32, [i32, vp, vp, i64]),
        "qo_vec_dot_f64": (f64, [i32, vp, vp, i64]),
        "qo_dot_f32_exact": (f32, [vp, vp, i64]),
        "qo_router_logits": (None, [vp, vp, i32, i32, i32, vp]),
        "qo_topk_softmax": (None, [vp, i32, i32, i32, vp, vp]),
        "qo_sort_assignments": (None, [vp, i32, i32, i32, vp, vp, vp]),
        "qo_silu_mul": (f32, [f32, f32]),
        "qo_sigmoid": (f32, [f32]),
        "qo_rms_norm": (None, [vp, vp, i32, i32, f32, vp]),
        "qo_rms_partials": (None, [vp, i32, i32, vp]),
        "qo_gelu_f16": (f32, [f32]),
        "qo_geglu_mul": (f32, [f32, f32]),
        "qo_gemma4_moe_inputs": (None, [vp, vp, vp, i32, i32, f32, vp, vp]),
        "qo_moe_forward": (i32, [ctypes.POINTER(QoLayer), vp, i32, vp, ctypes.POINTER(QoDebug), i32]),
        "qo_moe_forward_routed": (i32, [ctypes.POINTER(QoLayer), vp, vp, i32, vp, ctypes.POINTER(QoDebug), i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(type_id: int, n: int) -> int:
    return int(lib().qo_row_bytes(type_id, n))


# ---- vectorized helpers -------------------------------------------------------------
def gen_normal_f32(seed: int, stream: int, n: int, mean: float = 0.0, sigma: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().qo_gen_normal_f32(seed, stream, mean, sigma, _p(out), n)
    return out


def quantize(type_id: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * (18 if type_id == TYPE_Q4_0 else 34), dtype=np.uint8)
    fn = lib().qo_quantize_q4_0 if type_id == TYPE_Q4_0 else lib().qo_quantize_q8_0
    fn(_p(x), _p(out), x.size)
    return out


def quantize_act(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // 32 * 34, dtype=np.uint8)
    lib().qo_quantize_q8_0_act(_p(x), _p(out), x.size)
    return out


def dequantize(type_id: int, blocks: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().qo_dequantize(type_id, _p(np.ascontiguousarray(blocks)), _p(out), n)
    return out


def router_logits(w_router: np.ndarray, x: np.ndarray) -> np.ndarray:
    E, H = w_router.shape
    T = x.shape[0]
    out = np.empty((T, E), dtype=np.float32)
    lib().qo_router_logits(_p(np.ascontiguousarray(w_router)), _p(np.ascontiguousarray(x)), T, H, E, _p(out))
    return out


def topk_softmax(logits: np.ndarray, k: int):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    T, E = logits.shape
    idx = np.empty((T, k), dtype=np.int32)
    w = np.empty((T, k), dtype=np.float32)
    lib().qo_topk_softmax(_p(logits), T, E, k, _p(idx), _p(w))
    return idx, w


def sort_assignments(idx: np.ndarray, n_experts: int):
    idx = np.ascontiguousarray(idx, dtype=np.int32)
    T, k = idx.shape
    offsets = np.empty(n_experts + 1, dtype=np.int32)
    rows = np.empty(T * k, dtype=np.int32)
    pos = np.empty(T * k, dtype=np.int32)
    lib().qo_sort_assignments(_p(idx), T, n_experts, k, _p(offsets), _p(rows), _p(pos))
    return offsets, rows, pos


def rms_norm(x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H = x.shape
    y = np.empty_like(x)
    lib().qo_rms_norm(_p(x), _p(None if w is None else np.ascontiguousarray(w, dtype=np.float32)), T, H,
                      eps, _p(y))
    return y


def rms_partials(x: np.ndarray) -> np.ndarray:
    """qo_rms_partials: float64 [T, ceil(H/32)]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H = x.shape
    out = np.empty((T, (H + 31) // 32), dtype=np.float64)
    lib().qo_rms_partials(_p(x), T, H, _p(out))
    return out


ACT_SILU, ACT_GELU_TANH = 0, 1


def gelu_f16(x) -> np.ndarray:
    """ggml's CPU gelu (fp16 table semantics), elementwise."""
    x = np.asarray(x, dtype=np.float32)
    return np.array([lib().qo_gelu_f16(float(v)) for v in x.reshape(-1)], dtype=np.float32).reshape(x.shape)


def gemma4_moe_inputs(x: np.ndarray, w_pre: np.ndarray, w_rs: np.ndarray, eps: float):
    """(expert_in, router_in) of the Gemma 4 MoE branch from the residual rows x."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H = x.shape
    ei, ri = np.empty_like(x), np.empty_like(x)
    lib().qo_gemma4_moe_inputs(_p(x), _p(np.ascontiguousarray(w_pre, np.float32)),
                               _p(np.ascontiguousarray(w_rs, np.float32)), T, H, eps, _p(ei), _p(ri))
    return ei, ri


class Layer:
    """Host copy of one MoE layer in GGUF block layout (numpy uint8/float32).
    act: ACT_SILU (SwiGLU) or ACT_GELU_TANH (GeGLU); with tensors["gate_up"]
    (E x 2F rows: gate rows then up rows of each expert) instead of gate/up,
    the fused Gemma 4 layout."""

    def __init__(self, n_embd, n_experts, top_k, ffn_dim, shared, wtype, tensors: dict, act: int = ACT_SILU):
        self.H, self.E, self.K, self.F, self.S, self.wtype = n_embd, n_experts, top_k, ffn_dim, bool(shared), wtype
        self.act = act
        self.t = {k: np.ascontiguousarray(v) for k, v in tensors.items()}
        fused = "gate_up" in self.t
        names = ("router", "gate_up" if fused else "gate", "up", "down", "sh_gate", "sh_up", "sh_down", "sh_norm")
        self._c = QoLayer(n_embd, n_experts, top_k, ffn_dim, 1 if shared else 0, wtype,
                          *(_p(self.t.get(n)) for n in names), act, 1 if fused else 0)

    def forward(self, x: np.ndarray, nthreads: int = 0, debug: bool = False, router_in: np.ndarray | None = None):
        """y = MoE(x); the router reads router_in when given (else x)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        xr = x if router_in is None else np.ascontiguousarray(router_in, dtype=np.float32)
        assert xr.shape == x.shape
        T = x.shape[0]
        y = np.empty((T, self.H), dtype=np.float32)
        dbg = None
        d = None
        if debug:
            A = T * self.K
            d = {
                "logits": np.empty((T, self.E), np.float32), "topk_idx": np.empty((T, self.K), np.int32),
                "topk_w": np.empty((T, self.K), np.float32), "sh_gate": np.empty(T, np.float32),
                "offsets": np.empty(self.E + 1, np.int32), "rows": np.empty(A, np.int32),
                "h": np.empty((A, self.F), np.float32), "y": np.empty((A, self.H), np.float32),
                "sh_out": np.empty((T, self.H), np.float32), "sh_h": np.empty((T, self.F), np.float32),
            }
            dbg = QoDebug(*(_p(d[n]) for n in
                            ("logits", "topk_idx", "topk_w", "sh_gate", "offsets", "rows", "h", "y", "sh_out", "sh_h")))
        rc = lib().qo_moe_forward_routed(ctypes.byref(self._c), _p(x), _p(xr), T, _p(y),
                                         ctypes.byref(dbg) if dbg is not None else None, nthreads)
        if rc != 0:
            raise RuntimeError(f"qo_moe_forward failed with code {rc}")
        return (y, d) if debug else y


SLOTS = ("router", "gate", "up", "down", "sh_gate", "sh_up", "sh_down", "sh_norm")


def synth_layer(n_embd, n_experts, top_k, ffn_dim, shared, wtype, seed, layer=0, sigma=0.02,
                router_sigma=0.02, geglu=False) -> Layer:
    """CPU generation of the same recipe as qwenium_amd.synthetic.make_layer_tensors
    (geglu: the fused gate_up tensor and the GeGLU activation)."""
    H, E, F = n_embd, n_experts, ffn_dim
    sid = lambda slot: layer * 16 + SLOTS.index(slot)
    t = {"router": gen_normal_f32(seed, sid("router"), E * H, 0.0, router_sigma).reshape(E, H)}
    for slot in ("gate", "up"):
        t[slot] = quantize(wtype, gen_normal_f32(seed, sid(slot), E * F * H, 0.0, sigma))
    t["down"] = quantize(wtype, gen_normal_f32(seed, sid("down"), E * H * F, 0.0, sigma))
    if shared:
        for slot in ("sh_gate", "sh_up"):
            t[slot] = quantize(wtype, gen_normal_f32(seed, sid(slot), F * H, 0.0, sigma))
        t["sh_down"] = quantize(wtype, gen_normal_f32(seed, sid("sh_down"), H * F, 0.0, sigma))
        t["sh_norm"] = gen_normal_f32(seed, sid("sh_norm"), H, 0.0, router_sigma)
    if geglu:
        g, u = t.pop("gate").reshape(E, -1), t.pop("up").reshape(E, -1)
        t["gate_up"] = np.concatenate([g, u], axis=1).reshape(-1)
        return Layer(H, E, top_k, F, shared, wtype, t, act=ACT_GELU_TANH)
    return Layer(H, E, top_k, F, shared, wtype, t)


def synth_x(n_tokens: int, n_embd: int, seed: int, batch: int = 0) -> np.ndarray:
    return gen_normal_f32(seed, (1 << 40) + batch, n_tokens * n_embd).reshape(n_tokens, n_embd)
