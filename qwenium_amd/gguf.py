"""GGUF ingestion for the MoE layer over libqmoe's C ABI (qmoe_gguf_*).

Reference behaviour mirrored:
  GGUFLoader::load_model / get_tensor_data   src/loader/gguf_loader.cpp:46-91, 621-639
  raw_kv lookups of the MoE hparams          src/models/qwen36.cpp:23-25, 44-53, 97-102
  per-block MoE tensor binding               src/core/model.cpp:233-255 (names in
                                             src/models/qwen36.cpp:543-547)
  Gemma 4 MoE tensors and hparams             src/models/gemma4.cpp:96-98, 211-215, 297-303

The GGUF block layout is the layer's input layout, so tensors are copied to
the device byte for byte and wrapped as ggml views; nothing is repacked.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from ._lib import QmoeGgufTensor, QmoeTensor, check, lib
from .moe import GeGLUMoELayer, GGMLTensor, Hparams, MoELayer

# MoE tensors of block i ("blk.<i>." + name), in the layer's slot order
MOE_SLOTS = (
    ("router", "ffn_gate_inp.weight"),
    ("gate", "ffn_gate_exps.weight"),
    ("up", "ffn_up_exps.weight"),
    ("down", "ffn_down_exps.weight"),
    ("sh_gate", "ffn_gate_shexp.weight"),
    ("sh_up", "ffn_up_shexp.weight"),
    ("sh_down", "ffn_down_shexp.weight"),
    ("sh_norm", "ffn_gate_inp_shexp.weight"),
)
# Pre-MoE RMSNorm weight of a block (called post_attention_norm in the qwen35moe family, model.cpp:233-235)
FFN_NORM = "post_attention_norm.weight"
# Gemma 4 MoE tensors of block i (gemma4.cpp:211-215, 300-303) and its two MoE-branch norms
GEMMA4_MOE_SLOTS = (
    ("router", "ffn_gate_inp.weight"),
    ("gate_up", "ffn_gate_up_exps.weight"),
    ("down", "ffn_down_exps.weight"),
)
GEMMA4_PRE_NORM = "pre_ffw_norm_2.weight"
GEMMA4_ROUTER_SCALE = "ffn_gate_inp.scale"


class GGUFFile:
    """A memory-mapped GGUF file: metadata, tensor inventory, uploads."""

    def __init__(self, path: str):
        h = ctypes.c_void_p()
        check(lib().qmoe_gguf_open(path.encode(), ctypes.byref(h)))
        self._handle = h
        self.path = path

    def close(self) -> None:
        if getattr(self, "_handle", None):
            lib().qmoe_gguf_close(self._handle)
            self._handle = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # --- metadata -----------------------------------------------------------
    def info(self) -> dict:
        v, nt, nk, off = ctypes.c_uint32(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_uint64()
        check(lib().qmoe_gguf_info(self._handle, ctypes.byref(v), ctypes.byref(nt), ctypes.byref(nk), ctypes.byref(off)))
        return {"version": v.value, "n_tensors": nt.value, "n_kv": nk.value, "data_offset": off.value}

    def get_u32(self, key: str) -> int:
        v = ctypes.c_uint32()
        check(lib().qmoe_gguf_get_u32(self._handle, key.encode(), ctypes.byref(v)))
        return v.value

    def get_f32(self, key: str) -> float:
        v = ctypes.c_float()
        check(lib().qmoe_gguf_get_f32(self._handle, key.encode(), ctypes.byref(v)))
        return v.value

    def get_str(self, key: str) -> str:
        v = ctypes.c_char_p()
        check(lib().qmoe_gguf_get_str(self._handle, key.encode(), ctypes.byref(v)))
        return v.value.decode()

    # --- tensors -------------------------------------------------------------
    def tensor_names(self) -> list:
        n = self.info()["n_tensors"]
        out = []
        for i in range(n):
            p = ctypes.c_char_p()
            check(lib().qmoe_gguf_tensor_name(self._handle, i, ctypes.byref(p)))
            out.append(p.value.decode())
        return out

    def find(self, name: str) -> QmoeGgufTensor:
        t = QmoeGgufTensor()
        check(lib().qmoe_gguf_find(self._handle, name.encode(), ctypes.byref(t)))
        return t

    def has(self, name: str) -> bool:
        return name in set(self.tensor_names())

    def read(self, name: str) -> bytes:
        t = self.find(name)
        buf = ctypes.create_string_buffer(int(t.nbytes))
        check(lib().qmoe_gguf_read(self._handle, name.encode(), buf, t.nbytes))
        return buf.raw

    def upload(self, name: str, device="cuda") -> GGMLTensor:
        """Copies tensor `name` to `device` and returns it as a ggml view."""
        t = self.find(name)
        ne = tuple(int(t.ne[d]) for d in range(int(t.n_dims)))
        if t.type == 0:  # F32
            data = torch.empty(int(t.nbytes) // 4, dtype=torch.float32, device=device)
        else:
            data = torch.empty(int(t.nbytes), dtype=torch.uint8, device=device)
        stream = torch.cuda.current_stream(data.device).cuda_stream
        check(lib().qmoe_gguf_upload(self._handle, name.encode(), ctypes.c_void_p(data.data_ptr()), t.nbytes,
                                     ctypes.c_void_p(stream)))
        return GGMLTensor(data, int(t.type), ne)

    # --- the MoE block -------------------------------------------------------
    def moe_hparams(self, arch: Optional[str] = None, block: int = 0) -> Hparams:
        """{arch}.expert_count / expert_used_count / expert_feed_forward_length
        (qwen36.cpp:23-25, checked as at :44-53); the shared expert is present
        when the block has its tensors."""
        arch = arch or self.get_str("general.architecture")
        E = self.get_u32(f"{arch}.expert_count")
        K = self.get_u32(f"{arch}.expert_used_count")
        F = self.get_u32(f"{arch}.expert_feed_forward_length")
        if E == 0:
            raise ValueError(f'field "expert_count" expected > 0, got 0 (GGUF key: {arch}.expert_count)')
        if F == 0:
            raise ValueError(f'field "expert_feed_forward_length" expected > 0, got 0 '
                             f"(GGUF key: {arch}.expert_feed_forward_length)")
        if K > E:
            raise ValueError(f'field "expert_used_count" expected <= expert_count ({E}), got {K}')
        names = set(self.tensor_names())
        shared = f"blk.{block}.ffn_gate_shexp.weight" in names
        return Hparams(int(E), int(K), int(F), shared)

    def moe_tensors(self, block: int, device="cuda", shared: Optional[bool] = None) -> dict:
        """Uploads block `block`'s MoE tensors; keys as synthetic.make_layer_tensors."""
        names = set(self.tensor_names())
        out = {}
        for slot, suffix in MOE_SLOTS:
            name = f"blk.{block}.{suffix}"
            if slot.startswith("sh_") and (shared is False or name not in names):
                if shared:
                    raise ValueError(f"qwen35moe: missing tensor '{name}': expected in block weights, got absent")
                continue
            if name not in names:
                raise ValueError(f"qwen35moe: missing tensor '{name}': expected in block weights, got absent")
            out[slot] = self.upload(name, device)
        return out

    def moe_layer(self, block: int, device="cuda", prefill_copies: bool = False) -> MoELayer:
        """MoELayer of block `block` (weights uploaded; the layer keeps them alive);
        prefill_copies as MoELayer's (opt-in)."""
        hp = self.moe_hparams(block=block)
        t = self.moe_tensors(block, device, shared=hp.has_shared_expert)
        layer = MoELayer(t["router"], t["gate"], t["up"], t["down"], t.get("sh_gate"), t.get("sh_up"),
                         t.get("sh_down"), t.get("sh_norm"), hp, prefill_copies=prefill_copies)
        return layer

    def ffn_norm(self, block: int, device="cuda") -> torch.Tensor:
        """The block's pre-MoE RMSNorm weight [n_embd] f32."""
        return self.upload(f"blk.{block}.{FFN_NORM}", device).data

    def gemma4_moe_layer(self, block: int, device="cuda", prefill_copies: bool = False) -> GeGLUMoELayer:
        """GeGLUMoELayer of Gemma 4 block `block` (gemma4.* hparams, fused gate_up);
        prefill_copies as GeGLUMoELayer's (opt-in)."""
        hp = self.moe_hparams(arch="gemma4", block=block)
        names = set(self.tensor_names())
        t = {}
        for slot, suffix in GEMMA4_MOE_SLOTS:
            name = f"blk.{block}.{suffix}"
            if name not in names:
                raise ValueError(f"gemma4: missing tensor '{name}': expected in block weights, got absent")
            t[slot] = self.upload(name, device)
        return GeGLUMoELayer(t["router"], t["gate_up"], t["down"], hp, prefill_copies=prefill_copies)

    def gemma4_moe_norms(self, block: int, device="cuda"):
        """(pre_ffw_norm_2, ffn_gate_inp.scale) of Gemma 4 block `block`, [n_embd] f32 each."""
        return (self.upload(f"blk.{block}.{GEMMA4_PRE_NORM}", device).data,
                self.upload(f"blk.{block}.{GEMMA4_ROUTER_SCALE}", device).data)


def tensor_view(t: QmoeGgufTensor, device_ptr: int) -> QmoeTensor:
    """qmoe_gguf_tensor_view: the contiguous ggml view of an uploaded tensor."""
    v = QmoeTensor()
    check(lib().qmoe_gguf_tensor_view(ctypes.byref(t), ctypes.c_void_p(device_ptr), ctypes.byref(v)))
    return v
