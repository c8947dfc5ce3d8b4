"""The C ABI without a GPU: libqmoe.so loads, exports every function that
include/qmoe.h declares, and validates arguments on the host with the
reference's fail-loud contract ("<slot> expected <value>, got <value>";
src/qinf_error.h:1-29) and MoELayer's one constructor check
(src/layers/moe.cpp:47-52).  Descriptors carry fake (never dereferenced)
device pointers: validation reads only shapes, types and alignment."""
import ctypes
import os
import re

import pytest

from qwenium_amd import _lib
from qwenium_amd._lib import (QMOE_ERR_CAPACITY, QMOE_ERR_NULL, QMOE_ERR_SHAPE, QMOE_ERR_TYPE, QMOE_ERR_VALUE,
                              QMOE_OK, TYPE_F32, TYPE_Q4_0, TYPE_Q8_0, QmoeHparams, make_tensor)

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "qmoe.h")
FAKE = 0x10000000


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qmoe_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_function_is_exported():
    L = _lib.lib()
    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(L, n), f"{n} declared in include/qmoe.h but not exported"
    assert sorted(_lib.EXPORTED) == names


def layer_descs(H=2048, E=256, F=512, wt=TYPE_Q4_0, shared=True, ptr=FAKE):
    d = {
        "router": make_tensor(ptr, TYPE_F32, (H, E)),
        "gate": make_tensor(ptr, wt, (H, F, E)),
        "up": make_tensor(ptr, wt, (H, F, E)),
        "down": make_tensor(ptr, wt, (F, H, E)),
    }
    if shared:
        d.update({"sh_gate": make_tensor(ptr, wt, (H, F)), "sh_up": make_tensor(ptr, wt, (H, F)),
                  "sh_down": make_tensor(ptr, wt, (F, H)), "sh_norm": make_tensor(ptr, TYPE_F32, (H,))})
    return d


def create(d, hp):
    L = _lib.lib()
    order = ("router", "gate", "up", "down", "sh_gate", "sh_up", "sh_down", "sh_norm")
    args = [ctypes.byref(d[k]) if d.get(k) is not None else None for k in order]
    h = ctypes.c_void_p()
    rc = L.qmoe_layer_create(*args, ctypes.byref(hp), ctypes.byref(h))
    msg = _lib.last_error()
    if rc == QMOE_OK:
        L.qmoe_layer_destroy(h)
    return rc, msg


def test_valid_layer_creates():
    assert create(layer_descs(), QmoeHparams(256, 8, 512, 1)) == (QMOE_OK, "")
    assert create(layer_descs(1024, 16, 512, TYPE_Q8_0, False), QmoeHparams(16, 2, 512, 0))[0] == QMOE_OK


def test_shared_expert_null_weights_reference_message():
    d = layer_descs()
    d["sh_up"] = None
    rc, msg = create(d, QmoeHparams(256, 8, 512, 1))
    assert rc == QMOE_ERR_NULL
    assert msg == "moe_layer: has_shared_expert=true but shared expert weights are null"


@pytest.mark.parametrize("hp,needle", [
    (QmoeHparams(256, 0, 512, 1), '"top_k"'),
    (QmoeHparams(256, 300, 512, 1), '"top_k"'),
    (QmoeHparams(0, 8, 512, 1), '"n_experts"'),
    (QmoeHparams(256, 8, 500, 1), '"ffn_dim"'),
])
def test_bad_hparams(hp, needle):
    rc, msg = create(layer_descs(), hp)
    assert rc == QMOE_ERR_VALUE and needle in msg and "expected" in msg and "got" in msg


def test_expert_type_f32_rejected_with_slot_name():
    d = layer_descs()
    d["gate"] = make_tensor(FAKE, TYPE_F32, (2048, 512, 256))
    rc, msg = create(d, QmoeHparams(256, 8, 512, 1))
    assert rc == QMOE_ERR_TYPE
    assert msg.startswith('qmoe: slot "w_exp_gate" expected type Q4_0 or Q8_0, got F32')


def test_up_type_must_match_gate():
    d = layer_descs()
    d["up"] = make_tensor(FAKE, TYPE_Q8_0, (2048, 512, 256))
    rc, msg = create(d, QmoeHparams(256, 8, 512, 1))
    assert rc == QMOE_ERR_TYPE and '"w_exp_up"' in msg


def test_shape_mismatch_names_slot():
    d = layer_descs()
    d["down"] = make_tensor(FAKE, TYPE_Q4_0, (512, 1024, 256))
    rc, msg = create(d, QmoeHparams(256, 8, 512, 1))
    assert rc == QMOE_ERR_SHAPE and '"w_exp_down"' in msg and "ne[1]=2048" in msg


def test_router_width_rules():
    rc, msg = create(layer_descs(H=300), QmoeHparams(256, 8, 512, 1))
    assert rc == QMOE_ERR_SHAPE and '"w_router"' in msg


@pytest.mark.parametrize("H,F,slot", [(4128, 512, '"w_router"'), (2048, 100, '"ffn_dim"'),
                                      (2048, 4160, '"ffn_dim"'), (16, 512, '"w_router"')])
def test_widths_outside_the_limits_rejected(H, F, slot):
    """Widths that are not whole Q4_0/Q8_0 blocks (multiples of 32) or exceed 4096:
    rejected before any allocation or launch, naming the slot and the limit.  (Other
    multiples of 32 run on zero-padded weight copies: GPU tests.)"""
    rc, msg = create(layer_descs(H=H, F=F), QmoeHparams(256, 8, F, 1))
    assert rc in (QMOE_ERR_SHAPE, QMOE_ERR_VALUE)
    assert slot in msg and "multiple of" in msg and "got" in msg


def test_null_data_and_misaligned():
    d = layer_descs()
    d["gate"] = make_tensor(0, TYPE_Q4_0, (2048, 512, 256))
    assert create(d, QmoeHparams(256, 8, 512, 1))[0] == QMOE_ERR_NULL
    d = layer_descs()
    d["gate"] = make_tensor(FAKE + 2, TYPE_Q4_0, (2048, 512, 256))
    rc, msg = create(d, QmoeHparams(256, 8, 512, 1))
    assert rc == QMOE_ERR_SHAPE and "aligned" in msg


def test_short_row_stride_rejected():
    d = layer_descs()
    t = make_tensor(FAKE, TYPE_Q4_0, (2048, 512, 256), nb=(18, 1000, 1000 * 512))
    d["gate"] = t
    rc, msg = create(d, QmoeHparams(256, 8, 512, 1))
    assert rc == QMOE_ERR_SHAPE and "nb[1]" in msg


def test_forward_argument_checks_without_gpu():
    L = _lib.lib()
    assert L.qmoe_layer_forward(None, None, None, 1, None, None, None, None) == QMOE_ERR_NULL
    d = layer_descs()
    order = ("router", "gate", "up", "down", "sh_gate", "sh_up", "sh_down", "sh_norm")
    h = ctypes.c_void_p()
    hp = QmoeHparams(256, 8, 512, 1)
    assert L.qmoe_layer_create(*[ctypes.byref(d[k]) for k in order], ctypes.byref(hp), ctypes.byref(h)) == QMOE_OK
    try:
        assert L.qmoe_layer_n_embd(h) == 2048
        assert L.qmoe_layer_forward(h, None, FAKE, 0, FAKE, None, None, None) == QMOE_OK  # no-op, no GPU call
        assert L.qmoe_layer_forward(h, None, FAKE, -1, FAKE, None, None, None) == QMOE_ERR_VALUE
        assert L.qmoe_layer_forward(h, None, None, 4, FAKE, None, None, None) == QMOE_ERR_NULL
        assert L.qmoe_layer_forward(h, None, FAKE, 4, FAKE, None, None, None) == QMOE_ERR_VALUE  # y aliases x
        assert "distinct" in _lib.last_error()
        assert L.qmoe_layer_forward(h, None, FAKE + 4, 4, FAKE + 0x1000, None, None, None) == QMOE_ERR_VALUE
        assert "aligned" in _lib.last_error()
        assert L.qmoe_layer_set_phase_events(h, None) == QMOE_OK
    finally:
        L.qmoe_layer_destroy(h)
    assert L.qmoe_layer_set_phase_events(None, None) == QMOE_ERR_NULL


def test_workspace_and_misc_checks_without_gpu():
    L = _lib.lib()
    ws = ctypes.c_void_p()
    assert L.qmoe_workspace_create(None, 16, ctypes.byref(ws)) == QMOE_ERR_NULL
    assert L.qmoe_workspace_capacity(None) == 0
    assert L.qmoe_workspace_check(None, None) == 1  # QMOE_ERR_NULL
    assert L.qmoe_rms_norm(FAKE, None, 0, 2048, 1e-6, FAKE, None) == QMOE_OK
    assert L.qmoe_rms_norm(None, None, 3, 2048, 1e-6, FAKE, None) == QMOE_ERR_NULL
    assert L.qmoe_rms_partials(FAKE, 0, 2048, FAKE, None) == QMOE_OK
    assert L.qmoe_rms_partials(None, 3, 2048, FAKE, None) == QMOE_ERR_NULL
    assert L.qmoe_rms_partials(FAKE, 3, 0, FAKE, None) == QMOE_ERR_VALUE
    assert L.qmoe_rms_partials(FAKE, 3, 2048, FAKE + 4, None) == QMOE_ERR_VALUE
    assert L.qmoe_layer_forward_norm_chain(None, None, FAKE, None, FAKE, 1e-6, 4, FAKE + 0x1000, None, None,
                                           None) == QMOE_ERR_NULL  # no layer
    assert L.qmoe_layer_forward_norm_chain(None, None, FAKE, None, None, 1e-6, 4, FAKE + 0x1000, None, None,
                                           None) == QMOE_ERR_NULL  # no norm_w
    assert L.qmoe_layer_forward_norm_chain(None, None, FAKE, FAKE + 8, FAKE, 1e-6, 4, FAKE + 0x1000, None, None,
                                           None) == QMOE_ERR_VALUE
    assert "aligned" in _lib.last_error()
    assert L.qmoe_synth_quant(FAKE, TYPE_F32, 4, 64, 0, 0, 0.02, None) == QMOE_ERR_TYPE
    assert L.qmoe_synth_quant(FAKE, TYPE_Q4_0, 4, 40, 0, 0, 0.02, None) == QMOE_ERR_VALUE
    assert L.qmoe_synth_f32(FAKE, 0, 0, 0, 0.0, 1.0, None) == QMOE_OK
    assert QMOE_ERR_CAPACITY == 5


def test_python_wrapper_raises_with_message():
    from qwenium_amd import QmoeError
    with pytest.raises(QmoeError, match="has_shared_expert=true"):
        _lib.check(create({**layer_descs(), "sh_gate": None}, QmoeHparams(256, 8, 512, 1))[0])


# ---- the Python mirror's argument checks (no GPU: the checks run before any launch) ----

def test_python_row_and_vector_checks():
    import torch

    from qwenium_amd import moe

    dev = torch.device("cpu")
    x = torch.zeros(4, 8)
    ok = torch.zeros(4, 8)
    assert moe._rows_out("out", ok, 4, 8, dev, x) is ok
    for bad in (torch.zeros(3, 8), torch.zeros(4, 8, dtype=torch.float64), torch.zeros(8, 4).t(),
                torch.zeros(4 * 8), "not a tensor"):
        with pytest.raises(ValueError, match="out expected a contiguous"):
            moe._rows_out("out", bad, 4, 8, dev, x)
    with pytest.raises(ValueError, match="distinct from the input rows"):
        moe._rows_out("out", x, 4, 8, dev, x)
    # a read-only operand is copied when strided, rejected when the shape or type is wrong
    strided = torch.zeros(8, 4).t()
    assert moe._rows_in("residual", strided, 4, 8, dev).is_contiguous()
    for bad in (torch.zeros(4, 7), torch.zeros(4, 8, dtype=torch.float16), None):
        with pytest.raises(ValueError, match="residual expected"):
            moe._rows_in("residual", bad, 4, 8, dev)
    assert moe._vec_in("norm_weight", torch.zeros(8), 8, dev).shape == (8,)
    for bad in (torch.zeros(7), torch.zeros(1, 8), torch.zeros(8, dtype=torch.int32)):
        with pytest.raises(ValueError, match="norm_weight expected"):
            moe._vec_in("norm_weight", bad, 8, dev)
    # another device than the input rows'
    with pytest.raises(ValueError, match="on meta"):
        moe._rows_in("residual", torch.zeros(4, 8), 4, 8, torch.device("meta"))


def test_python_forward_rejects_host_input():
    import torch

    from qwenium_amd import moe

    layer = moe.MoELayer.__new__(moe.MoELayer)  # no handle: the checks fail before any call into the library
    layer.n_embd = 8
    with pytest.raises(ValueError, match="x expected a cuda float32"):
        layer.forward(torch.zeros(2, 8))
    with pytest.raises(ValueError, match="x expected a cuda float32"):
        layer.forward_norm(torch.zeros(2, 8), torch.ones(8), 1e-6)
    with pytest.raises(ValueError, match="x expected a cuda float32"):
        moe.rms_norm(torch.zeros(2, 8), None, 1e-6)
