"""The allocation-free forward (qmoe_layer_forward_static): through the C ABI,
against qmoe_layer_forward on a workspace of its own, bit for bit, on two calls
in a row with the second one smaller; and its size limit, checked on the host."""
import ctypes

import numpy as np
import pytest

from qwenium_amd import _lib
from qwenium_amd._lib import QMOE_ERR_CAPACITY, QMOE_OK, TYPE_F32, TYPE_Q4_0, QmoeHparams, make_tensor


def test_static_forward_rejects_sizes_above_the_scratch():
    """Host-side check before any device work (fake device pointers, never dereferenced)."""
    L = _lib.lib()
    H, E, F, FAKE = 2048, 256, 512, 0x10000000
    d = [make_tensor(FAKE, TYPE_F32, (H, E)), make_tensor(FAKE, TYPE_Q4_0, (H, F, E)),
         make_tensor(FAKE, TYPE_Q4_0, (H, F, E)), make_tensor(FAKE, TYPE_Q4_0, (F, H, E)),
         make_tensor(FAKE, TYPE_Q4_0, (H, F)), make_tensor(FAKE, TYPE_Q4_0, (H, F)),
         make_tensor(FAKE, TYPE_Q4_0, (F, H)), make_tensor(FAKE, TYPE_F32, (H,))]
    h = ctypes.c_void_p()
    assert L.qmoe_layer_create(*(ctypes.byref(t) for t in d), ctypes.byref(QmoeHparams(E, 8, F, 1)),
                               ctypes.byref(h)) == QMOE_OK
    try:
        rc = L.qmoe_layer_forward_static(h, FAKE, 4096, FAKE, None, None)
        assert rc == QMOE_ERR_CAPACITY
        assert "static scratch" in _lib.last_error() and "4096 tokens" in _lib.last_error()
        assert L.qmoe_layer_forward_static(h, FAKE, 0, FAKE, None, None) == QMOE_OK  # no-op
    finally:
        L.qmoe_layer_destroy(h)


@pytest.mark.gpu
@pytest.mark.parametrize("spec_name,sizes", [("QWEN35B", (40, 3)), ("QWEN35B", (10, 1)), ("CONFIG1", (32, 17)),
                                             ("GEMMA4", (16, 5)), ("PADDED", (20, 3)), ("LISTS", (300, 130))])
def test_static_forward_matches_workspace_forward(gpu, spec_name, sizes):
    import torch

    from qwenium_amd import Workspace, synthetic
    from qwenium_amd._lib import check, lib

    # PADDED: widths off the kernels' grid (the static scratch also holds the padded rows);
    # LISTS: 300 tokens over 256 experts take the per-expert list launch and the MFMA GEMMs with
    # their fixup list, then 130 tokens the merged top-k and the streaming GEMVs on the same scratch
    spec = (synthetic.LayerSpec(96, 8, 2, 32, True, synthetic.TYPE_Q4_0) if spec_name == "PADDED"
            else synthetic.LayerSpec(256, 256, 8, 64, True, synthetic.TYPE_Q4_0) if spec_name == "LISTS"
            else getattr(synthetic, spec_name))
    layer = synthetic.make_layer(spec, 29)
    ws = Workspace(layer, max(sizes))
    stream = torch.cuda.current_stream().cuda_stream
    for i, T in enumerate(sizes):
        x = synthetic.make_x(spec, T, 29, batch=i)
        res = synthetic.make_x(spec, T, 30, batch=i) if i == 0 else None
        want = layer.forward(x, residual=res, workspace=ws)
        got = torch.full_like(x, float("nan"))
        check(lib().qmoe_layer_forward_static(layer._handle, x.data_ptr(), T, got.data_ptr(),
                                              res.data_ptr() if res is not None else None, stream))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"{spec_name} T={T}"
        assert np.isfinite(got.cpu().numpy()).all()
    assert ws.check() == 0
