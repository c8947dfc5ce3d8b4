"""qwenium_amd -- MI355X-native (gfx950) MoE FFN layer for Qwenium-style models.

The compute path is libqmoe.so: hand-written HIP kernels behind the C ABI of
include/qmoe.h.  This package is its Python host mirror (ctypes) plus seeded
synthetic-layer helpers; torch provides device memory and streams only.
"""
from ._lib import (QMOE_ERR_CAPACITY, QMOE_ERR_HIP, QMOE_ERR_NULL, QMOE_ERR_SHAPE, QMOE_ERR_TYPE,
                   QMOE_ERR_VALUE, QMOE_OK, TYPE_F32, TYPE_Q4_0, TYPE_Q8_0, QmoeError, lib)
from .moe import (GeGLUMoELayer, GGMLTensor, Hparams, MoELayer, Phase, Workspace, gelu_f16_table, gemma4_moe_inputs,
                  rms_norm, rms_partials, ssq_parts, synth_f32, synth_quant)
from .telemetry import MoEMetrics, MoEResidencyTracker

__all__ = [
    "GeGLUMoELayer", "GGMLTensor", "Hparams", "MoELayer", "gelu_f16_table", "gemma4_moe_inputs", "MoEMetrics", "MoEResidencyTracker", "Phase", "Workspace", "rms_norm", "rms_partials", "ssq_parts", "synth_f32", "synth_quant",
    "QmoeError", "lib", "TYPE_F32", "TYPE_Q4_0", "TYPE_Q8_0", "QMOE_OK", "QMOE_ERR_NULL", "QMOE_ERR_SHAPE",
    "QMOE_ERR_TYPE", "QMOE_ERR_VALUE", "QMOE_ERR_CAPACITY", "QMOE_ERR_HIP",
]
