"""Seeded synthetic MoE layers in GGUF block layout, generated on the device.

Tensor values follow the workload definitions: router / shared gate f32
N(0, 0.02); expert and shared matrices N(0, 0.02) quantized with ggml's
reference quantizers; activations N(0, 1).  Each tensor has its own RNG stream
(seed, stream id), and value i of a stream is a pure function of
(seed, stream, i), so a CPU implementation of the same recipe reproduces the
exact bytes (the tests check that).
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch

from ._lib import TYPE_F32, TYPE_Q4_0, TYPE_Q8_0, row_bytes
from .moe import GeGLUMoELayer, GGMLTensor, Hparams, MoELayer, synth_f32, synth_quant

SLOTS = ("router", "gate", "up", "down", "sh_gate", "sh_up", "sh_down", "sh_norm")


def stream_id(layer: int, slot: str) -> int:
    return layer * 16 + SLOTS.index(slot)


def x_stream(batch: int) -> int:
    """RNG stream of activation batch `batch`."""
    return (1 << 40) + batch


@dataclasses.dataclass(frozen=True)
class Skew:
    """Routing skew by construction (a shared direction u = 1/sqrt(H) in every
    coordinate): x += c*u and router row e += beta_e*u, so logit e gains the
    constant c*beta_e (plus beta_e*(z.u), N(0, beta_e^2) per token).  Experts
    are ranked by a seeded permutation; rank r (1-based) gets bias
    c*beta = -a*s*ln(r) (a Zipf(s) log-profile) and the last `n_empty` ranks
    get `empty_bias` (never selected).  a = 0.6 puts ~50% of a 2048-token
    batch's top-8 assignments on the 8 hot experts, with ~46 experts empty."""
    s: float = 1.2
    a: float = 0.6
    n_empty: int = 40
    empty_bias: float = -40.0
    c: float = 8.0
    perm_seed: int = 7

    def biases(self, n_experts: int):
        import numpy as np

        rank_of = np.empty(n_experts, np.int64)
        rank_of[np.random.default_rng(self.perm_seed).permutation(n_experts)] = np.arange(1, n_experts + 1)
        b = -self.a * self.s * np.log(rank_of.astype(np.float64))
        b[rank_of > n_experts - self.n_empty] = self.empty_bias
        return b  # logit bias c*beta_e per expert id

    def hot_experts(self, n_experts: int, n: int = 8):
        import numpy as np

        return np.argsort(-self.biases(n_experts), kind="stable")[:n]


@dataclasses.dataclass
class LayerSpec:
    n_embd: int
    n_experts: int
    top_k: int
    ffn_dim: int
    shared: bool
    wtype: int = TYPE_Q4_0
    sigma: float = 0.02
    router_sigma: float = 0.02
    skew: Optional[Skew] = None
    geglu: bool = False  # Gemma 4 layout: fused gate_up tensor, GeGLU-tanh, router on its own input

    @property
    def hparams(self) -> Hparams:
        return Hparams(self.n_experts, self.top_k, self.ffn_dim, self.shared)


# The workloads (hidden, experts, top-k, ffn, shared, weight type).
CONFIG1 = LayerSpec(1024, 16, 2, 512, False, TYPE_Q8_0)       # ggml CPU-path case
QWEN35B = LayerSpec(2048, 256, 8, 512, True, TYPE_Q4_0)       # Qwen3.6-35B-A3B MoE layer
QWEN35B_Q8 = LayerSpec(2048, 256, 8, 512, True, TYPE_Q8_0)    # same shape, Q8_0 weights
QWEN35B_SKEW = LayerSpec(2048, 256, 8, 512, True, TYPE_Q8_0, skew=Skew())  # Zipf-skewed routing, Q8_0
# Gemma 4 26B-A4B MoE layer (gemma4.h:72,89-91: n_embd 2816, 128 experts, top-8, expert ffn 704)
GEMMA4 = LayerSpec(2816, 128, 8, 704, False, TYPE_Q4_0, geglu=True)
GEMMA4_Q8 = LayerSpec(2816, 128, 8, 704, False, TYPE_Q8_0, geglu=True)


def layer_bytes(spec: LayerSpec) -> dict:
    """Byte size of every tensor of one layer."""
    H, E, F = spec.n_embd, spec.n_experts, spec.ffn_dim
    rb_h = row_bytes(spec.wtype, H)
    rb_f = row_bytes(spec.wtype, F)
    out = {
        "router": E * H * 4,
        "gate": E * F * rb_h,
        "up": E * F * rb_h,
        "down": E * H * rb_f,
    }
    if spec.shared:
        out.update({"sh_gate": F * rb_h, "sh_up": F * rb_h, "sh_down": H * rb_f, "sh_norm": H * 4})
    return out


def make_layer_tensors(spec: LayerSpec, seed: int, layer: int = 0, device="cuda") -> dict:
    """Generates one layer's tensors on `device` as GGMLTensor views."""
    H, E, F, wt = spec.n_embd, spec.n_experts, spec.ffn_dim, spec.wtype
    t = {}
    router = synth_f32(E * H, seed, stream_id(layer, "router"), 0.0, spec.router_sigma, device=device)
    if spec.skew is not None:
        beta = torch.tensor(spec.skew.biases(E) / spec.skew.c / H ** 0.5, dtype=torch.float32, device=device)
        router = (router.view(E, H) + beta[:, None]).reshape(-1)
    t["router"] = GGMLTensor(router, TYPE_F32, (H, E))
    for slot in ("gate", "up"):
        t[slot] = GGMLTensor(synth_quant(wt, E * F, H, seed, stream_id(layer, slot), spec.sigma, device=device),
                             wt, (H, F, E))
    if spec.geglu:
        # one [H, 2F, E] tensor: each expert's gate rows, then its up rows (gemma4.cpp:397-409)
        rb = row_bytes(wt, H)
        g, u = t.pop("gate").data.view(E, F * rb), t.pop("up").data.view(E, F * rb)
        t["gate_up"] = GGMLTensor(torch.cat([g, u], dim=1).reshape(-1), wt, (H, 2 * F, E))
    t["down"] = GGMLTensor(synth_quant(wt, E * H, F, seed, stream_id(layer, "down"), spec.sigma, device=device),
                           wt, (F, H, E))
    if spec.shared:
        for slot in ("sh_gate", "sh_up"):
            t[slot] = GGMLTensor(synth_quant(wt, F, H, seed, stream_id(layer, slot), spec.sigma, device=device),
                                 wt, (H, F))
        t["sh_down"] = GGMLTensor(synth_quant(wt, H, F, seed, stream_id(layer, "sh_down"), spec.sigma,
                                              device=device), wt, (F, H))
        t["sh_norm"] = GGMLTensor(synth_f32(H, seed, stream_id(layer, "sh_norm"), 0.0, spec.router_sigma,
                                            device=device), TYPE_F32, (H,))
    return t


def make_layer(spec: LayerSpec, seed: int, layer: int = 0, device="cuda",
               tensors: Optional[dict] = None, prefill_copies: bool = True) -> MoELayer:
    """The layer over seeded synthetic weights; prefill_copies: opt in to the
    chunk-major copies of the expert matrices (the faster prefill GEMMs)."""
    t = tensors if tensors is not None else make_layer_tensors(spec, seed, layer, device)
    if spec.geglu:
        return GeGLUMoELayer(t["router"], t["gate_up"], t["down"], spec.hparams, prefill_copies=prefill_copies)
    return MoELayer(t["router"], t["gate"], t["up"], t["down"], t.get("sh_gate"), t.get("sh_up"),
                    t.get("sh_down"), t.get("sh_norm"), spec.hparams, prefill_copies=prefill_copies)


def make_x(spec: LayerSpec, n_tokens: int, seed: int, batch: int = 0, device="cuda") -> torch.Tensor:
    x = synth_f32(n_tokens * spec.n_embd, seed, x_stream(batch), 0.0, 1.0, device=device).view(
        n_tokens, spec.n_embd)
    if spec.skew is not None:
        x = x + torch.tensor(spec.skew.c / spec.n_embd ** 0.5, dtype=torch.float32, device=device)
    return x


def norm_stream(layer: int) -> int:
    """RNG stream of the pre-MoE RMSNorm weight of stack layer `layer`."""
    return (1 << 41) + layer


def make_norm_weight(spec: LayerSpec, seed: int, layer: int, device="cuda") -> torch.Tensor:
    """Pre-MoE RMSNorm weight of a stack layer: N(1, 0.02)."""
    return synth_f32(spec.n_embd, seed, norm_stream(layer), 1.0, 0.02, device=device)


def make_gemma4_norms(spec: LayerSpec, seed: int, layer: int, device="cuda"):
    """(pre_ffw_norm_2, ffn_gate_inp.scale) of a Gemma 4 block: N(1, 0.02) each."""
    return (synth_f32(spec.n_embd, seed, (1 << 42) + 2 * layer, 1.0, 0.02, device=device),
            synth_f32(spec.n_embd, seed, (1 << 42) + 2 * layer + 1, 1.0, 0.02, device=device))


# Pre-MoE RMSNorm epsilon of the layer stack (qwen36.cpp:298 reads it from the GGUF; 1e-6 here).
NORM_EPS = 1e-6
