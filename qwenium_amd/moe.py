"""Python mirror of the reference's MoE layer module over libqmoe's C ABI.

Reference interface (rye-001/Qwenium):
  MoELayer::Hparams           src/layers/moe.h:34-39
  MoELayer::MoELayer(8 slots) src/layers/moe.h:44-53, src/layers/moe.cpp:27-53
  MoELayer::build(...)        src/layers/moe.h:58-63  -> MoELayer.forward here
  build_rms_norm(...)         src/layers/norm.cpp:15-26 -> rms_norm here
  Gemma4ForwardPass::build_moe_geglu  src/models/gemma4.cpp:367-445 -> GeGLUMoELayer

torch supplies device memory and the current HIP stream only; every
computation runs in libqmoe's HIP kernels.
"""
from __future__ import annotations

import contextlib
import ctypes
import dataclasses
import os
from typing import Optional

import torch

from . import _lib
from ._lib import TYPE_F32, TYPE_Q4_0, TYPE_Q8_0, QmoeDebug, QmoeHparams, check, lib, make_tensor, row_bytes


class Phase:
    """layer.h:19-22; accepted by forward() for interface symmetry and ignored."""
    Prefill = 0
    Decode = 1


@dataclasses.dataclass
class Hparams:
    n_experts: int
    top_k: int
    ffn_dim: int
    has_shared_expert: bool


@dataclasses.dataclass
class GGMLTensor:
    """A device tensor in ggml/GGUF layout: raw bytes (uint8) or f32 data plus
    the ggml type id and ne (ne[0] contiguous)."""
    data: torch.Tensor
    type: int
    ne: tuple

    def desc(self) -> _lib.QmoeTensor:
        if not self.data.is_contiguous():
            raise ValueError("GGMLTensor.data must be contiguous")
        return make_tensor(self.data.data_ptr(), self.type, tuple(self.ne))


def _stream_ptr(stream) -> Optional[int]:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def _on(stream):
    """Makes `stream` current while the arguments of a launch are prepared, so
    contiguous copies and output allocations are ordered on the stream the
    kernels run on (and return to its pool when freed)."""
    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


def _rows_in(name: str, t: torch.Tensor, T: int, H: int, device) -> torch.Tensor:
    """A read-only [T, H] f32 operand on `device` (the input rows' device, a
    cuda device once x has been checked): checked, then made contiguous."""
    if (not isinstance(t, torch.Tensor) or t.dim() != 2 or tuple(t.shape) != (T, H) or t.dtype != torch.float32
            or t.device != device):
        raise ValueError(f"{name} expected a cuda float32 [{T}, {H}] tensor on {device}, got "
                         f"{_describe(t)}")
    return t.contiguous()


def _rows_out(name: str, t: Optional[torch.Tensor], T: int, H: int, device, like: torch.Tensor) -> torch.Tensor:
    """The [T, H] f32 output: a new tensor, or the caller's, which must be
    contiguous (the kernels write T*H floats from its first element)."""
    if t is None:
        return torch.empty((T, H), dtype=torch.float32, device=device)
    if (not isinstance(t, torch.Tensor) or t.dim() != 2 or tuple(t.shape) != (T, H) or t.dtype != torch.float32
            or t.device != device or not t.is_contiguous()):
        raise ValueError(f"{name} expected a contiguous cuda float32 [{T}, {H}] tensor on {device}, got "
                         f"{_describe(t)}")
    if t.data_ptr() == like.data_ptr():
        raise ValueError(f"{name} expected a buffer distinct from the input rows, got the same storage")
    return t


def _vec_in(name: str, t: torch.Tensor, H: int, device) -> torch.Tensor:
    """A per-feature f32 weight [H] on `device`."""
    if (not isinstance(t, torch.Tensor) or t.dim() != 1 or t.shape[0] != H or t.dtype != torch.float32
            or t.device != device):
        raise ValueError(f"{name} expected a cuda float32 [{H}] tensor on {device}, got {_describe(t)}")
    return t.contiguous()


def ssq_parts(n_embd: int) -> int:
    """Entries per row of the RMSNorm partial sums (32 columns each)."""
    return (n_embd + 31) // 32


def _ssq_in(name: str, t: torch.Tensor, T: int, H: int, device) -> torch.Tensor:
    if (not isinstance(t, torch.Tensor) or tuple(t.shape) != (T, ssq_parts(H)) or t.dtype != torch.float64
            or t.device != device):
        raise ValueError(f"{name} expected a cuda float64 [{T}, {ssq_parts(H)}] tensor on {device}, got "
                         f"{_describe(t)}")
    return t.contiguous()


def _ssq_out(name: str, t: torch.Tensor, T: int, H: int, device) -> torch.Tensor:
    if (not isinstance(t, torch.Tensor) or tuple(t.shape) != (T, ssq_parts(H)) or t.dtype != torch.float64
            or t.device != device or not t.is_contiguous()):
        raise ValueError(f"{name} expected a contiguous cuda float64 [{T}, {ssq_parts(H)}] tensor on {device}, got "
                         f"{_describe(t)}")
    return t


def _describe(t) -> str:
    if not isinstance(t, torch.Tensor):
        return type(t).__name__
    return f"{tuple(t.shape)} {t.dtype} on {t.device}{'' if t.is_contiguous() else ' (non-contiguous)'}"


class Workspace:
    """Scratch for up to max_tokens tokens of layers no larger than `like`."""

    def __init__(self, like: "MoELayer", max_tokens: int):
        h = ctypes.c_void_p()
        check(lib().qmoe_workspace_create(like._handle, int(max_tokens), ctypes.byref(h)))
        self._handle = h

    @property
    def capacity(self) -> int:
        return int(lib().qmoe_workspace_capacity(self._handle))

    def check(self) -> int:
        """Synchronizes (raising on a device error) and reports whether a forward on
        this workspace failed a cross-workgroup wait: always 0, since no kernel waits
        on another workgroup."""
        v = ctypes.c_int32()
        check(lib().qmoe_workspace_check(self._handle, ctypes.byref(v)))
        return int(v.value)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            lib().qmoe_workspace_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoELayer:
    """Same slot order and hparams as the reference's MoELayer constructor."""

    def __init__(self, w_router: GGMLTensor, w_exp_gate: GGMLTensor, w_exp_up: GGMLTensor,
                 w_exp_down: GGMLTensor, w_sh_gate: Optional[GGMLTensor], w_sh_up: Optional[GGMLTensor],
                 w_sh_down: Optional[GGMLTensor], w_sh_norm: Optional[GGMLTensor], hp: Hparams, *,
                 prefill_copies: bool = False):
        self.hp = hp
        # keep the borrowed weights alive for the layer's lifetime
        self._weights = (w_router, w_exp_gate, w_exp_up, w_exp_down, w_sh_gate, w_sh_up, w_sh_down, w_sh_norm)
        descs = [w.desc() if w is not None else None for w in self._weights]
        ptrs = [ctypes.byref(d) if d is not None else None for d in descs]
        c_hp = QmoeHparams(int(hp.n_experts), int(hp.top_k), int(hp.ffn_dim), 1 if hp.has_shared_expert else 0)
        h = ctypes.c_void_p()
        check(lib().qmoe_layer_create(*ptrs, ctypes.byref(c_hp), ctypes.byref(h)))
        self._handle = h
        self.n_embd = int(lib().qmoe_layer_n_embd(h))
        self._maybe_prefill_copies(prefill_copies, w_exp_gate)

    def _maybe_prefill_copies(self, wanted: bool, probe: GGMLTensor) -> None:
        # the copies read the weights now: only for device-resident tensors, and not
        # when QMOE_PREFILL_REPACK=0 (the prefill GEMMs then read the GGUF rows)
        if wanted and probe.data.is_cuda and os.environ.get("QMOE_PREFILL_REPACK", "1") != "0":
            self.build_prefill_copies()

    def build_prefill_copies(self) -> None:
        """Chunk-major copies of the expert matrices for the prefill GEMMs, opt-in: one more
        copy of the expert weights in device memory (455 MB for a 35B-A3B layer in Q4_0,
        18.2 GB for its 40 layers); reads the tensors now.  Without them the prefill GEMMs
        read the GGUF rows: the same results, slower prefill."""
        check(lib().qmoe_layer_build_prefill_copies(self._handle))

    def close(self) -> None:
        if getattr(self, "_handle", None):
            lib().qmoe_layer_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_expert_counts(self, counts: Optional[torch.Tensor]) -> None:
        """Attaches a device dispatch histogram: while set, every forward adds
        its per-expert dispatch counts (T*top_k in total) to `counts`, a cuda
        int64 [n_experts] tensor (read as u64), on the forward's stream.  None
        detaches it.  The layer keeps the tensor alive while attached."""
        if counts is not None:
            if (counts.dtype != torch.int64 or not counts.is_cuda or counts.dim() != 1
                    or counts.shape[0] != self.hp.n_experts or not counts.is_contiguous()):
                raise ValueError(f"counts expected a contiguous cuda int64 [{self.hp.n_experts}] tensor, got "
                                 f"{tuple(counts.shape)} {counts.dtype} on {counts.device}")
        check(lib().qmoe_layer_set_expert_counts(self._handle, counts.data_ptr() if counts is not None else None))
        self._expert_counts = counts

    def forward(self, x: torch.Tensor, phase: int = Phase.Prefill, il: int = 0, *,
                residual: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                workspace: Optional[Workspace] = None, debug: bool = False, stream=None):
        """y[T][n_embd] = MoE(x) (+ residual).  With debug=True also returns the
        routing intermediates (logits, topk_idx, topk_w, sh_gate, offsets, rows, and
        router_approx/router_bound, left NaN unless the batched MFMA router ran)."""
        del phase, il  # MoE has one topology (moe.h:55-57); il only names tensors in ggml
        with _on(stream):
            x = self._check_x(x)
            T = x.shape[0]
            res = _rows_in("residual", residual, T, self.n_embd, x.device) if residual is not None else None
            y = _rows_out("out", out, T, self.n_embd, x.device, x)
            dbg, dbg_tensors = self._debug(T, x.device, debug) if debug else (None, None)
            check(lib().qmoe_layer_forward(
                self._handle, workspace._handle if workspace is not None else None,
                x.data_ptr(), int(T), y.data_ptr(), res.data_ptr() if res is not None else None,
                ctypes.byref(dbg) if dbg is not None else None, _stream_ptr(stream)))
        return (y, dbg_tensors) if debug else y

    def forward_norm(self, x: torch.Tensor, norm_weight: torch.Tensor, eps: float, *,
                     out: Optional[torch.Tensor] = None, workspace: Optional[Workspace] = None,
                     x_ssq: Optional[torch.Tensor] = None, y_ssq: Optional[torch.Tensor] = None,
                     debug: bool = False, stream=None):
        """The block's caller slice in one call (qwen36.cpp:297-304):
        y = x + MoE(RMSNorm(x) * norm_weight).  Same bits as
        forward(rms_norm(x, norm_weight, eps), residual=x).  For a chain of
        blocks, x_ssq may hold x's RMSNorm partial sums (rms_partials(x), or
        the previous block's y_ssq) and y_ssq receives y's: float64
        [T, ceil(n_embd/32)] (qmoe_layer_forward_norm_chain); the bits do not
        change."""
        with _on(stream):
            x = self._check_x(x)
            T = x.shape[0]
            w = _vec_in("norm_weight", norm_weight, self.n_embd, x.device)
            y = _rows_out("out", out, T, self.n_embd, x.device, x)
            dbg, dbg_tensors = self._debug(T, x.device, debug) if debug else (None, None)
            ws = workspace._handle if workspace is not None else None
            d = ctypes.byref(dbg) if dbg is not None else None
            if x_ssq is None and y_ssq is None:
                check(lib().qmoe_layer_forward_norm(self._handle, ws, x.data_ptr(), w.data_ptr(), float(eps), int(T),
                                                    y.data_ptr(), d, _stream_ptr(stream)))
            else:
                xs = _ssq_in("x_ssq", x_ssq, T, self.n_embd, x.device) if x_ssq is not None else None
                ys = _ssq_out("y_ssq", y_ssq, T, self.n_embd, x.device) if y_ssq is not None else None
                check(lib().qmoe_layer_forward_norm_chain(
                    self._handle, ws, x.data_ptr(), xs.data_ptr() if xs is not None else None, w.data_ptr(),
                    float(eps), int(T), y.data_ptr(), ys.data_ptr() if ys is not None else None, d,
                    _stream_ptr(stream)))
        return (y, dbg_tensors) if debug else y

    def forward_routed(self, expert_in: torch.Tensor, router_in: torch.Tensor, *, out: Optional[torch.Tensor] = None,
                       workspace: Optional[Workspace] = None, debug: bool = False, stream=None):
        """y = MoE(expert_in) routed on router_in (build_moe_geglu's two inputs,
        gemma4.cpp:367-380); the shared expert's gate, if any, reads router_in."""
        with _on(stream):
            x = self._check_x(expert_in)
            xr = _rows_in("router_in", router_in, x.shape[0], self.n_embd, x.device)
            y = _rows_out("out", out, x.shape[0], self.n_embd, x.device, x)
            if y.data_ptr() == xr.data_ptr():
                raise ValueError("out expected a buffer distinct from router_in, got the same storage")
            dbg, dbg_tensors = self._debug(x.shape[0], x.device, debug) if debug else (None, None)
            check(lib().qmoe_layer_forward_routed(
                self._handle, workspace._handle if workspace is not None else None, x.data_ptr(), xr.data_ptr(),
                int(x.shape[0]), y.data_ptr(), ctypes.byref(dbg) if dbg is not None else None,
                _stream_ptr(stream)))
        return (y, dbg_tensors) if debug else y

    def _check_x(self, x: torch.Tensor) -> torch.Tensor:
        if (not isinstance(x, torch.Tensor) or x.dim() != 2 or x.shape[1] != self.n_embd
                or x.dtype != torch.float32 or not x.is_cuda):
            raise ValueError(f"x expected a cuda float32 [T, {self.n_embd}] tensor, got {_describe(x)}")
        return x.contiguous()

    def _debug(self, T: int, dev, what=True):
        """Device buffers for the forward's intermediates: the routing (logits,
        topk_idx, topk_w, sh_gate, offsets, rows, router_approx/router_bound),
        h's Q8_0 as the down projection reads it (h_qs [R, ffn_dim] int8, h_d
        [R, ffn_dim/32] scales; R = T*top_k assignment rows, then one shared row
        per token) and h_fixed (h blocks recomputed exactly on the MFMA path);
        with what == "rows" also exp_down [R, n_embd], the unweighted expert rows
        (left NaN where the combine consumes them in registers)."""
        E, k, F = self.hp.n_experts, self.hp.top_k, self.hp.ffn_dim
        R = T * k + (T if self.hp.has_shared_expert else 0)
        t = {
            "logits": torch.empty((T, E), dtype=torch.float32, device=dev),
            "topk_idx": torch.empty((T, k), dtype=torch.int32, device=dev),
            "topk_w": torch.empty((T, k), dtype=torch.float32, device=dev),
            "sh_gate": torch.empty((T,), dtype=torch.float32, device=dev),
            "offsets": torch.empty((E + 1,), dtype=torch.int32, device=dev),
            "rows": torch.empty((T * k,), dtype=torch.int32, device=dev),
            "router_approx": torch.full((T, E), float("nan"), dtype=torch.float32, device=dev),
            "router_bound": torch.full((T, E), float("nan"), dtype=torch.float32, device=dev),
            "h_qs": torch.empty((R, F), dtype=torch.int8, device=dev),
            "h_d": torch.empty((R, F // 32), dtype=torch.float32, device=dev),
            "h_fixed": torch.full((1,), -1, dtype=torch.int32, device=dev),
        }
        if what == "rows":
            t["exp_down"] = torch.full((R, self.n_embd), float("nan"), dtype=torch.float32, device=dev)
        names = ("logits", "topk_idx", "topk_w", "sh_gate", "offsets", "rows", "router_approx", "router_bound",
                 "h_qs", "h_d", "h_fixed", "exp_down")
        dbg = QmoeDebug(*(t[n].data_ptr() if n in t else None for n in names))
        return dbg, t

    __call__ = forward


class GeGLUMoELayer(MoELayer):
    """Gemma 4's MoE (Gemma4ForwardPass::build_moe_geglu, gemma4.cpp:367-445):
    the fused gate_up tensor [n_embd, 2*ffn_dim, n_experts], GeGLU-tanh
    (ggml's CPU gelu), no shared expert, the router on its own input."""

    def __init__(self, w_router: GGMLTensor, w_gate_up_exps: GGMLTensor, w_down_exps: GGMLTensor, hp: Hparams, *,
                 prefill_copies: bool = False):
        if hp.has_shared_expert:
            raise ValueError("has_shared_expert expected False for the GeGLU MoE, got True")
        self.hp = hp
        self._weights = (w_router, w_gate_up_exps, w_down_exps)
        descs = [w.desc() for w in self._weights]
        c_hp = QmoeHparams(int(hp.n_experts), int(hp.top_k), int(hp.ffn_dim), 0)
        h = ctypes.c_void_p()
        check(lib().qmoe_geglu_layer_create(*(ctypes.byref(d) for d in descs), ctypes.byref(c_hp), ctypes.byref(h)))
        self._handle = h
        self.n_embd = int(lib().qmoe_layer_n_embd(h))
        self._maybe_prefill_copies(prefill_copies, w_gate_up_exps)

    def forward_gemma4(self, x: torch.Tensor, pre_norm_weight: torch.Tensor, router_scale: torch.Tensor, eps: float,
                       *, out: Optional[torch.Tensor] = None, workspace: Optional[Workspace] = None,
                       debug: bool = False, stream=None):
        """The Gemma 4 MoE branch from the residual rows x (gemma4.cpp:555-565):
        build_moe_geglu(rms_norm(x)*pre_norm_weight, (rms_norm(x)/sqrt(n_embd))*router_scale)."""
        with _on(stream):
            x = self._check_x(x)
            w = _vec_in("pre_norm_weight", pre_norm_weight, self.n_embd, x.device)
            rs = _vec_in("router_scale", router_scale, self.n_embd, x.device)
            y = _rows_out("out", out, x.shape[0], self.n_embd, x.device, x)
            dbg, dbg_tensors = self._debug(x.shape[0], x.device, debug) if debug else (None, None)
            check(lib().qmoe_layer_forward_gemma4(
                self._handle, workspace._handle if workspace is not None else None, x.data_ptr(), w.data_ptr(),
                rs.data_ptr(), float(eps), int(x.shape[0]), y.data_ptr(),
                ctypes.byref(dbg) if dbg is not None else None, _stream_ptr(stream)))
        return (y, dbg_tensors) if debug else y


def gemma4_moe_inputs(x: torch.Tensor, pre_norm_weight: torch.Tensor, router_scale: torch.Tensor, eps: float,
                      stream=None):
    """(expert_in, router_in) of the Gemma 4 MoE branch (gemma4.cpp:555-563)."""
    with _on(stream):
        if not isinstance(x, torch.Tensor) or x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda:
            raise ValueError(f"x expected a cuda float32 [T, n_embd] tensor, got {_describe(x)}")
        x = x.contiguous()
        w = _vec_in("pre_norm_weight", pre_norm_weight, x.shape[1], x.device)
        rs = _vec_in("router_scale", router_scale, x.shape[1], x.device)
        ei, ri = torch.empty_like(x), torch.empty_like(x)
        check(lib().qmoe_gemma4_moe_inputs(x.data_ptr(), w.data_ptr(), rs.data_ptr(), float(eps), int(x.shape[0]),
                                           int(x.shape[1]), ei.data_ptr(), ri.data_ptr(), _stream_ptr(stream)))
    return ei, ri


def gelu_f16_table():
    """The 65536-entry fp16 gelu table of the GeGLU kernels (numpy uint16)."""
    import numpy as np

    out = np.empty(65536, dtype=np.uint16)
    check(lib().qmoe_gelu_f16_table(out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16))))
    return out


def rms_norm(x: torch.Tensor, w: Optional[torch.Tensor], eps: float, out: Optional[torch.Tensor] = None,
             stream=None) -> torch.Tensor:
    """build_rms_norm (norm.cpp:15-26): x / sqrt(mean(x^2) + eps) * w, per token."""
    with _on(stream):
        if not isinstance(x, torch.Tensor) or x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda:
            raise ValueError(f"x expected a cuda float32 [T, n_embd] tensor, got {_describe(x)}")
        x = x.contiguous()
        T, H = x.shape
        wc = _vec_in("w", w, H, x.device) if w is not None else None
        y = _rows_out("out", out, T, H, x.device, x) if out is not None else torch.empty_like(x)
        check(lib().qmoe_rms_norm(x.data_ptr(), wc.data_ptr() if wc is not None else None, int(T), int(H),
                                  float(eps), y.data_ptr(), _stream_ptr(stream)))
    return y


def rms_partials(x: torch.Tensor, out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    """rms_norm's sum of squares of each row of x in pieces of 32 columns
    (float64 [T, ceil(n_embd/32)]; qmoe_rms_partials)."""
    with _on(stream):
        if not isinstance(x, torch.Tensor) or x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda:
            raise ValueError(f"x expected a cuda float32 [T, n_embd] tensor, got {_describe(x)}")
        x = x.contiguous()
        T, H = x.shape
        y = (_ssq_out("out", out, T, H, x.device) if out is not None else
             torch.empty((T, ssq_parts(H)), dtype=torch.float64, device=x.device))
        check(lib().qmoe_rms_partials(x.data_ptr(), int(T), int(H), y.data_ptr(), _stream_ptr(stream)))
    return y


def synth_f32(n: int, seed: int, stream_id: int, mean: float = 0.0, sigma: float = 1.0,
              device="cuda", out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    y = out if out is not None else torch.empty((n,), dtype=torch.float32, device=device)
    check(lib().qmoe_synth_f32(y.data_ptr(), int(n), int(seed), int(stream_id), float(mean), float(sigma),
                               _stream_ptr(stream)))
    return y


def synth_quant(type_id: int, n_rows: int, row_len: int, seed: int, stream_id: int, sigma: float,
                device="cuda", out: Optional[torch.Tensor] = None, stream=None) -> torch.Tensor:
    nbytes = n_rows * row_bytes(type_id, row_len)
    y = out if out is not None else torch.empty((nbytes,), dtype=torch.uint8, device=device)
    check(lib().qmoe_synth_quant(y.data_ptr(), int(type_id), int(n_rows), int(row_len), int(seed),
                                 int(stream_id), float(sigma), _stream_ptr(stream)))
    return y
