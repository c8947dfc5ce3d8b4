"""Writes tests/golden/config1_seed0.npz: the CPU oracle's outputs for the
ggml-CPU-path workload (hidden 1024, 16 experts, top-2, ffn 512, no shared
expert, Q8_0 weights from N(0,0.02), f32 router N(0,0.02), 32 tokens of
N(0,1) activations, seed 0).  Inputs are regenerated from the seed by the
tests; SHA-256 digests of the weight and input bytes pin the generator.

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import pyoracle as po  # noqa: E402

H, E, K, F, T, SEED = 1024, 16, 2, 512, 32, 0


def make_inputs():
    layer = po.synth_layer(H, E, K, F, False, po.TYPE_Q8_0, seed=SEED)
    x = po.synth_x(T, H, seed=SEED)
    return layer, x


def digests(layer, x):
    out = {k: hashlib.sha256(np.ascontiguousarray(v).tobytes()).hexdigest() for k, v in layer.t.items()}
    out["x"] = hashlib.sha256(x.tobytes()).hexdigest()
    return out


def main():
    layer, x = make_inputs()
    y, d = layer.forward(x, debug=True)
    dg = digests(layer, x)
    path = os.path.join(HERE, "config1_seed0.npz")
    np.savez_compressed(path, y=y, logits=d["logits"], topk_idx=d["topk_idx"], topk_w=d["topk_w"],
                        offsets=d["offsets"], rows=d["rows"],
                        digest_names=np.array(sorted(dg)), digest_values=np.array([dg[k] for k in sorted(dg)]))
    print(path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
