"""Committed golden vectors for the ggml-CPU-path workload (hidden 1024, 16
experts, top-2, ffn 512, Q8_0, 32 tokens, seed 0): the oracle must keep
reproducing them, and the generator must keep producing the same bytes."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

import make_golden  # noqa: E402

FIXTURE = os.path.join(HERE, "golden", "config1_seed0.npz")


def test_generator_digests_and_oracle_outputs():
    ref = np.load(FIXTURE, allow_pickle=False)
    layer, x = make_golden.make_inputs()
    dg = make_golden.digests(layer, x)
    assert dict(zip(ref["digest_names"].tolist(), ref["digest_values"].tolist())) == dg
    y, d = layer.forward(x, debug=True)
    np.testing.assert_array_equal(d["topk_idx"], ref["topk_idx"])
    np.testing.assert_array_equal(d["offsets"], ref["offsets"])
    np.testing.assert_array_equal(d["rows"], ref["rows"])
    np.testing.assert_array_equal(d["logits"].view(np.int32), ref["logits"].view(np.int32))
    np.testing.assert_array_equal(d["topk_w"].view(np.int32), ref["topk_w"].view(np.int32))
    np.testing.assert_array_equal(y.view(np.int32), ref["y"].view(np.int32))


def test_fixture_invariants():
    ref = np.load(FIXTURE, allow_pickle=False)
    idx = ref["topk_idx"]
    assert idx.shape == (32, 2)
    assert np.all(idx[:, 0] != idx[:, 1])
    np.testing.assert_allclose(ref["topk_w"].sum(1), 1.0, rtol=1e-6)
    assert np.all(ref["topk_w"][:, 0] >= ref["topk_w"][:, 1])
    assert ref["offsets"][-1] == 64 and np.all(np.diff(ref["offsets"]) >= 0)
    assert sorted(ref["rows"].tolist()) == list(range(64))
