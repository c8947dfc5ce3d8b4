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
from .moe import GGMLTensor, Hparams, MoELayer, synth_f32, synth_quant

SLOTS = ("router", "gate", "up", "down", "sh_gate", "sh_up", "sh_down", "sh_norm")


def stream_id(layer: int, slot: str) -> int:
    return layer * 16 + SLOTS.index(slot)


def x_stream(batch: int) -> int:
    """RNG stream of activation batch `batch`."""
    return (1 << 40) + batch


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

    @property
    def hparams(self) -> Hparams:
        return Hparams(self.n_experts, self.top_k, self.ffn_dim, self.shared)


# The workloads (hidden, experts, top-k, ffn, shared, weight type).
CONFIG1 = LayerSpec(1024, 16, 2, 512, False, TYPE_Q8_0)       # ggml CPU-path case
QWEN35B = LayerSpec(2048, 256, 8, 512, True, TYPE_Q4_0)       # Qwen3.6-35B-A3B MoE layer
QWEN35B_Q8 = LayerSpec(2048, 256, 8, 512, True, TYPE_Q8_0)    # same shape, Q8_0 weights


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
    t["router"] = GGMLTensor(synth_f32(E * H, seed, stream_id(layer, "router"), 0.0, spec.router_sigma,
                                       device=device), TYPE_F32, (H, E))
    for slot in ("gate", "up"):
        t[slot] = GGMLTensor(synth_quant(wt, E * F, H, seed, stream_id(layer, slot), spec.sigma, device=device),
                             wt, (H, F, E))
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
               tensors: Optional[dict] = None) -> MoELayer:
    t = tensors if tensors is not None else make_layer_tensors(spec, seed, layer, device)
    return MoELayer(t["router"], t["gate"], t["up"], t["down"], t.get("sh_gate"), t.get("sh_up"),
                    t.get("sh_down"), t.get("sh_norm"), spec.hparams)


def make_x(spec: LayerSpec, n_tokens: int, seed: int, batch: int = 0, device="cuda") -> torch.Tensor:
    return synth_f32(n_tokens * spec.n_embd, seed, x_stream(batch), 0.0, 1.0, device=device).view(
        n_tokens, spec.n_embd)
