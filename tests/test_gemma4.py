"""Gemma 4 GeGLU MoE (Gemma4ForwardPass::build_moe_geglu, src/models/gemma4.cpp:367-445).

CPU: the oracle's gelu pinned against the reference's own GeGLU test
(tests/unit/test_ffn.cpp:131-177), against the double-precision tanh formula
over every fp16 input, against its thresholds and odd symmetry, and against the
wrong variants (erf form, sigmoid form); libqmoe's fp16 table against the
oracle entry by entry; the oracle's fused gate_up layout and separate router
input against the unfused oracle; the Gemma 4 input prep against RMSNorm.

GPU: the HIP path through the C ABI against the oracle on the same seeded
inputs at the 26B-A4B shape (n_embd 2816, 128 experts, top-8, ffn 704) over
the decode, streaming and MFMA paths, with the bar of the Qwen layer: routing
bit-exact, outputs within 2e-3 x RMS and in practice bit-identical.
"""
import math

import numpy as np
import pytest

from oracle import pyoracle as po
from qwenium_amd import TYPE_Q4_0, TYPE_Q8_0

TOL = 2e-3


def gelu_tanh_double(x):
    # the reference test's hand-computed oracle (test_ffn.cpp:131-136), in double
    return 0.5 * x * (1.0 + math.tanh(0.7978845608028654 * (x + 0.044715 * x ** 3)))


def all_fp16_in_range():
    h = np.arange(65536, dtype=np.uint16)
    f = h.view(np.float16).astype(np.float32)
    keep = np.isfinite(f) & (f > -10) & (f < 10)
    return h[keep], f[keep]


# ---- the oracle's gelu --------------------------------------------------------------

def test_gelu_reference_kat():
    """test_ffn.cpp:149-177: ggml's gelu within 1e-3 of the tanh formula at 8 points."""
    for x in (-2.0, -1.0, -0.5, 0.0, 0.25, 0.5, 1.0, 2.0):
        assert abs(po.lib().qo_gelu_f16(x) - gelu_tanh_double(x)) <= 1e-3, x


def test_gelu_every_fp16_input_within_one_fp16_ulp():
    """Over every fp16 x in (-10, 10): the oracle equals fp16(gelu(x)) computed in
    double to within one fp16 spacing plus the f32 cancellation of 1 + tanhf(z)
    for negative x (absolute 0.5*|x|*2^-23: ggml's f32 formula, reproduced, not
    corrected), and exactly in all but a few entries where no cancellation occurs."""
    _, f = all_fp16_in_range()
    got = po.gelu_f16(f)
    exact = np.array([gelu_tanh_double(float(v)) for v in f], dtype=np.float64)
    want = exact.astype(np.float16).astype(np.float32)
    spacing = np.maximum(np.abs(np.spacing(want.astype(np.float16))),
                         np.abs(np.spacing(got.astype(np.float16)))).astype(np.float64)
    cancel = np.where(f < 0, 0.5 * np.abs(f.astype(np.float64)) * 2.0 ** -23, 0.0)
    assert np.all(np.abs(got.astype(np.float64) - want) <= spacing + cancel)
    assert np.mean(got != want) < 1e-2
    assert np.mean((got != want)[f > -2]) < 1e-3


def test_gelu_thresholds_and_rounding_of_input():
    g = po.lib().qo_gelu_f16
    assert g(-10.0) == 0.0 and g(-1e6) == 0.0
    assert g(10.0) == 10.0 and g(12.3) == np.float32(12.3)
    # inside (-10, 10) the input is rounded to fp16 first: 1 + 2^-12 reads as 1
    assert g(1.0 + 2.0 ** -12) == g(1.0)
    assert g(9.999) == np.float32(np.float16(gelu_tanh_double(float(np.float16(9.999)))))


def test_gelu_identity_and_wrong_variants():
    """gelu(x) - gelu(-x) = x (Phi(x) + Phi(-x) = 1) up to fp16 rounding; the erf
    form and the sigmoid form (x*sigmoid(1.702x)) differ from it by more than an
    fp16 spacing somewhere on the KAT points."""
    for x in np.linspace(-6, 6, 97, dtype=np.float32):
        x16 = float(np.float16(x))
        d = po.lib().qo_gelu_f16(x16) - po.lib().qo_gelu_f16(-x16)
        assert abs(d - x16) <= 2 * abs(float(np.spacing(np.float16(x16)))) + 1e-7
    pts = np.array([-2.0, -1.0, -0.5, 0.25, 0.5, 1.0, 2.0], np.float32)
    ours = po.gelu_f16(pts)
    sp = np.abs(np.spacing(ours.astype(np.float16))).astype(np.float64)
    erf_form = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in pts])
    sig_form = np.array([v / (1 + math.exp(-1.702 * v)) for v in pts])
    assert np.any(np.abs(erf_form - ours) > sp)
    assert np.any(np.abs(sig_form - ours) > 10 * sp)


# ---- libqmoe's table -------------------------------------------------------------------

def test_library_gelu_table_matches_oracle_bit_for_bit():
    from qwenium_amd import gelu_f16_table

    tab = gelu_f16_table()
    h, f = all_fp16_in_range()
    want = np.array([po.lib().qo_fp32_to_fp16(po.lib().qo_gelu_f16(float(v))) for v in f], dtype=np.uint16)
    np.testing.assert_array_equal(tab[h], want)
    # non-finite codes map to themselves
    codes = np.arange(65536, dtype=np.uint16)
    nonfin = ~np.isfinite(codes.view(np.float16))
    np.testing.assert_array_equal(tab[nonfin], codes[nonfin])


# ---- the oracle's layer variants -----------------------------------------------------

def small_pair(act, seed=3, H=256, E=8, K=2, F=64, wtype=TYPE_Q8_0):
    unfused = po.synth_layer(H, E, K, F, False, wtype, seed)
    fused = po.synth_layer(H, E, K, F, False, wtype, seed, geglu=True)
    unfused = po.Layer(H, E, K, F, False, wtype, unfused.t, act=act)
    return unfused, fused


def test_oracle_fused_gate_up_equals_separate_tensors():
    """The fused [H, 2F, E] layout (gate rows then up rows per expert) gives the
    bits of the separate gate/up tensors; swapping the halves does not."""
    unfused, fused = small_pair(po.ACT_GELU_TANH)
    x = po.gen_normal_f32(5, 1, 12 * 256).reshape(12, 256)
    y0, d0 = unfused.forward(x, debug=True)
    y1, d1 = fused.forward(x, debug=True)
    np.testing.assert_array_equal(y0.view(np.uint32), y1.view(np.uint32))
    np.testing.assert_array_equal(d0["h"].view(np.uint32), d1["h"].view(np.uint32))
    E, F = 8, 64
    g, u = unfused.t["gate"].reshape(E, -1), unfused.t["up"].reshape(E, -1)
    swapped = dict(fused.t, gate_up=np.concatenate([u, g], axis=1).reshape(-1))
    ys = po.Layer(256, E, 2, F, False, TYPE_Q8_0, swapped, act=po.ACT_GELU_TANH).forward(x)
    assert not np.array_equal(ys, y1)


def test_oracle_geglu_h_is_gelu_times_up():
    _, fused = small_pair(po.ACT_GELU_TANH)
    x = po.gen_normal_f32(6, 1, 4 * 256).reshape(4, 256)
    _, d = fused.forward(x, debug=True)
    silu = po.Layer(256, 8, 2, 64, False, TYPE_Q8_0, fused.t, act=po.ACT_SILU)
    _, ds = silu.forward(x, debug=True)
    assert not np.array_equal(d["h"], ds["h"])
    # token 0's first expert, rows f: h = gelu(g) * u from the oracle's own block dots
    E, F, H = 8, 64, 256
    xq = po.quantize_act(x[0])
    rb = po.row_bytes(TYPE_Q8_0, H)
    gu = fused.t["gate_up"].reshape(E, 2 * F, rb)
    e = int(d["topk_idx"][0, 0])
    for f in (0, 17, 63):
        g = po.lib().qo_vec_dot(TYPE_Q8_0, po._p(np.ascontiguousarray(gu[e, f])), po._p(xq), H)
        u = po.lib().qo_vec_dot(TYPE_Q8_0, po._p(np.ascontiguousarray(gu[e, F + f])), po._p(xq), H)
        assert d["h"][0, f] == np.float32(po.lib().qo_gelu_f16(g)) * np.float32(u)


def test_oracle_router_input_separate():
    _, fused = small_pair(po.ACT_GELU_TANH)
    x = po.gen_normal_f32(7, 1, 9 * 256).reshape(9, 256)
    xr = po.gen_normal_f32(7, 2, 9 * 256).reshape(9, 256)
    y_same = fused.forward(x)
    np.testing.assert_array_equal(fused.forward(x, router_in=x), y_same)
    _, d = fused.forward(x, debug=True, router_in=xr)
    _, dr = fused.forward(xr, debug=True)
    np.testing.assert_array_equal(d["topk_idx"], dr["topk_idx"])  # routing follows router_in
    np.testing.assert_array_equal(d["logits"], dr["logits"])


def test_oracle_gemma4_inputs():
    """expert_in is RMSNorm(x)*w_pre (the pinned qo_rms_norm); router_in is
    ((RMSNorm(x)) * (1/sqrtf(H))) * w_rs in three f32 roundings."""
    T, H = 5, 2816
    x = po.gen_normal_f32(8, 1, T * H).reshape(T, H)
    w_pre = po.gen_normal_f32(8, 2, H, 1.0, 0.02)
    w_rs = po.gen_normal_f32(8, 3, H, 1.0, 0.02)
    ei, ri = po.gemma4_moe_inputs(x, w_pre, w_rs, 1e-6)
    np.testing.assert_array_equal(ei, po.rms_norm(x, w_pre, 1e-6))
    n = po.rms_norm(x, None, 1e-6)
    s = np.float32(1.0) / np.sqrt(np.float32(H))
    np.testing.assert_array_equal(ri, (n * s) * w_rs)


# ---- GPU -----------------------------------------------------------------------------

def host_layer(spec, tensors):
    host = {k: v.data.cpu().numpy() for k, v in tensors.items()}
    host["router"] = host["router"].reshape(spec.n_experts, spec.n_embd)
    return po.Layer(spec.n_embd, spec.n_experts, spec.top_k, spec.ffn_dim, False, spec.wtype, host,
                    act=po.ACT_GELU_TANH)


# bound on the f16-MFMA prefill path's error (T >= 128), as in test_gpu_parity
MFMA_TOL = 2e-5


def assert_parity(y, got, y_ref, d_ref, min_identical=0.999, mfma=False):
    np.testing.assert_array_equal(got["topk_idx"], d_ref["topk_idx"])
    np.testing.assert_array_equal(got["offsets"], d_ref["offsets"])
    np.testing.assert_array_equal(got["rows"], d_ref["rows"])
    ulp = np.abs(got["logits"].view(np.int32).astype(np.int64) - d_ref["logits"].view(np.int32).astype(np.int64))
    assert ulp.max() <= 1, f"router logits differ by {ulp.max()} ulp"
    np.testing.assert_allclose(got["topk_w"], d_ref["topk_w"], rtol=1e-6, atol=0)
    if "h_qs" in got:
        # h's Q8_0 as the down projection reads it equals the oracle's, bit for bit
        h = d_ref["h"]
        if got["h_qs"].shape[0] > h.shape[0]:
            h = np.concatenate([h, d_ref["sh_h"]], axis=0)
        R, F = h.shape
        blocks = po.quantize_act(h).reshape(R, F // 32, 34)
        np.testing.assert_array_equal(got["h_qs"], blocks[:, :, 2:].copy().view(np.int8).reshape(R, F))
        np.testing.assert_array_equal(got["h_d"], blocks[:, :, :2].copy().view(np.float16)[..., 0].astype(np.float32))
    rms = float(np.sqrt(np.mean(y_ref.astype(np.float64) ** 2)))
    err = float(np.max(np.abs(y - y_ref)))
    assert err <= TOL * rms, f"max |y - y_ref| = {err:.3e} > {TOL} * rms ({rms:.3e})"
    identical = float(np.mean(y.view(np.int32) == y_ref.view(np.int32)))
    if mfma:
        assert err <= MFMA_TOL * rms, f"f16-MFMA path: max |y - y_ref| = {err / rms:.2e} x rms > {MFMA_TOL}"
    else:
        assert identical >= min_identical, f"only {identical:.5f} of outputs bit-identical"


@pytest.mark.gpu
@pytest.mark.parametrize("wname,T", [("GEMMA4", 1), ("GEMMA4", 10), ("GEMMA4", 16), ("GEMMA4", 17),
                                     ("GEMMA4", 100), ("GEMMA4", 200), ("GEMMA4", 300), ("GEMMA4", 700),
                                     ("GEMMA4", 4096), ("GEMMA4_Q8", 10), ("GEMMA4_Q8", 256)])
def test_gemma4_layer_matches_oracle(gpu, wname, T):
    """Decode (T <= 16: fused routing + gate/up + down/combine), streaming
    (17..127) and MFMA (>= 128; batched router from 272 at this shape) paths, from the Gemma 4
    inputs the GPU prepares, against the oracle fed the same inputs."""
    import torch

    from qwenium_amd import Workspace, gemma4_moe_inputs, synthetic

    spec = getattr(synthetic, wname)
    seed = 31 + T
    tensors = synthetic.make_layer_tensors(spec, seed)
    layer = synthetic.make_layer(spec, seed, tensors=tensors)
    x = synthetic.make_x(spec, T, seed)
    w_pre, w_rs = synthetic.make_gemma4_norms(spec, seed, 0)
    ei, ri = gemma4_moe_inputs(x, w_pre, w_rs, synthetic.NORM_EPS)
    ws = Workspace(layer, T)
    y, dbg = layer.forward_routed(ei, ri, workspace=ws, debug=True)
    y_one = layer.forward_gemma4(x, w_pre, w_rs, synthetic.NORM_EPS, workspace=ws)
    torch.cuda.synchronize()
    assert ws.check() == 0
    assert torch.equal(y, y_one), "one-call Gemma 4 slice differs from inputs + forward_routed"
    ref = host_layer(spec, tensors)
    y_ref, d_ref = ref.forward(ei.cpu().numpy(), debug=True, router_in=ri.cpu().numpy())
    got = {k: v.cpu().numpy() for k, v in dbg.items()}
    assert_parity(y.cpu().numpy(), got, y_ref, d_ref, mfma=T >= 128)


@pytest.mark.gpu
@pytest.mark.parametrize("T", [10, 40, 150])
def test_geglu_padded_widths(gpu, T):
    """A GeGLU layer at widths off the kernels' grid (n_embd 160, ffn_dim 96): the Gemma 4
    slice (inputs at the caller's width, then zero-padded) against the oracle."""
    import torch

    from qwenium_amd import Workspace, gemma4_moe_inputs, synthetic

    spec = synthetic.LayerSpec(160, 16, 4, 96, False, TYPE_Q4_0, geglu=True)
    seed = 61 + T
    tensors = synthetic.make_layer_tensors(spec, seed)
    layer = synthetic.make_layer(spec, seed, tensors=tensors)
    x = synthetic.make_x(spec, T, seed)
    w_pre, w_rs = synthetic.make_gemma4_norms(spec, seed, 0)
    ei, ri = gemma4_moe_inputs(x, w_pre, w_rs, synthetic.NORM_EPS)
    ws = Workspace(layer, T)
    y, dbg = layer.forward_routed(ei, ri, workspace=ws, debug=True)
    y_one = layer.forward_gemma4(x, w_pre, w_rs, synthetic.NORM_EPS, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(y, y_one)
    ref = host_layer(spec, tensors)
    y_ref, d_ref = ref.forward(ei.cpu().numpy(), debug=True, router_in=ri.cpu().numpy())
    got = {k: v.cpu().numpy() for k, v in dbg.items()}
    assert_parity(y.cpu().numpy(), got, y_ref, d_ref, mfma=T >= 128)


@pytest.mark.gpu
def test_gemma4_inputs_match_oracle(gpu):
    from qwenium_amd import gemma4_moe_inputs, synthetic

    spec = synthetic.GEMMA4
    x = synthetic.make_x(spec, 7, 5)
    w_pre, w_rs = synthetic.make_gemma4_norms(spec, 5, 3)
    ei, ri = gemma4_moe_inputs(x, w_pre, w_rs, 1e-6)
    e_ref, r_ref = po.gemma4_moe_inputs(x.cpu().numpy(), w_pre.cpu().numpy(), w_rs.cpu().numpy(), 1e-6)
    np.testing.assert_allclose(ei.cpu().numpy(), e_ref, rtol=2e-7, atol=0)
    np.testing.assert_allclose(ri.cpu().numpy(), r_ref, rtol=2e-7, atol=0)


@pytest.mark.gpu
def test_geglu_layer_forward_routes_on_x(gpu):
    """forward(x) of a GeGLU layer is forward_routed(x, x)."""
    import torch

    from qwenium_amd import synthetic

    spec = synthetic.GEMMA4
    layer = synthetic.make_layer(spec, 9)
    x = synthetic.make_x(spec, 10, 9)
    y0 = layer.forward(x)
    y1 = layer.forward_routed(x, x)
    torch.cuda.synchronize()
    assert torch.equal(y0, y1)


@pytest.mark.gpu
def test_routed_forward_on_qwen_layer(gpu):
    """A separate router input on the SwiGLU layer: routing follows router_in
    (the shared gate too), the experts read expert_in; against the oracle."""
    from qwenium_amd import synthetic

    spec = synthetic.LayerSpec(1024, 32, 4, 256, True, TYPE_Q4_0)
    tensors = synthetic.make_layer_tensors(spec, 4)
    layer = synthetic.make_layer(spec, 4, tensors=tensors)
    for T in (10, 40, 300):
        x = synthetic.make_x(spec, T, 4, batch=1)
        xr = synthetic.make_x(spec, T, 4, batch=2)
        y, dbg = layer.forward_routed(x, xr, debug=True)
        host = {k: v.data.cpu().numpy() for k, v in tensors.items()}
        host["router"] = host["router"].reshape(spec.n_experts, spec.n_embd)
        ref = po.Layer(spec.n_embd, spec.n_experts, spec.top_k, spec.ffn_dim, True, spec.wtype, host)
        y_ref, d_ref = ref.forward(x.cpu().numpy(), debug=True, router_in=xr.cpu().numpy())
        got = {k: v.cpu().numpy() for k, v in dbg.items()}
        assert_parity(y.cpu().numpy(), got, y_ref, d_ref, mfma=T >= 128)
        np.testing.assert_allclose(got["sh_gate"], d_ref["sh_gate"], rtol=1e-6, atol=0)


@pytest.mark.gpu
def test_geglu_layer_rejects_bad_inputs(gpu):
    import torch

    from qwenium_amd import GeGLUMoELayer, GGMLTensor, Hparams, QmoeError, synthetic

    spec = synthetic.GEMMA4
    t = synthetic.make_layer_tensors(spec, 2)
    with pytest.raises(ValueError):
        GeGLUMoELayer(t["router"], t["gate_up"], t["down"], Hparams(128, 8, 704, True))
    half = GGMLTensor(t["gate_up"].data, spec.wtype, (2816, 704, 128))  # not 2*ffn rows
    with pytest.raises(QmoeError, match="w_gate_up_exps"):
        GeGLUMoELayer(t["router"], half, t["down"], spec.hparams)
    layer = synthetic.make_layer(spec, 2, tensors=t)
    x = synthetic.make_x(spec, 4, 2)
    with pytest.raises(ValueError):
        layer.forward_routed(x, x[:3])
    torch.cuda.synchronize()


def _geglu_cases(n=16, seed=4042):
    """Seeded GeGLU layer shapes and token counts over every path (fixed at import)."""
    from qwenium_amd import synthetic
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        H = int(rng.choice([256, 512, 1056, 2816]))
        E = int(rng.choice([8, 16, 64, 128]))
        K = int(min(E, rng.choice([1, 2, 4, 8])))
        F = int(rng.choice([64, 96, 128, 704]))
        wtype = TYPE_Q4_0 if rng.integers(2) else TYPE_Q8_0
        T = int(rng.choice([1, 10, 17, 40, 130, 300]))
        cases.append(pytest.param(synthetic.LayerSpec(H, E, K, F, False, wtype, geglu=True), T,
                                  id=f"H{H}-E{E}-k{K}-F{F}-{'q4' if wtype == TYPE_Q4_0 else 'q8'}-T{T}"))
    return cases


@pytest.mark.gpu
@pytest.mark.parametrize("spec,T", _geglu_cases())
def test_geglu_random_shapes(gpu, spec, T):
    """Seeded random GeGLU shapes, the Gemma 4 slice against the oracle: routing bit-exact,
    outputs bit-identical below the MFMA threshold (max(128, 5.5 n_experts / top_k)
    tokens), within MFMA_TOL with exact h quants above it."""
    import torch

    from qwenium_amd import Workspace, gemma4_moe_inputs, synthetic

    seed = 90 + T
    tensors = synthetic.make_layer_tensors(spec, seed)
    layer = synthetic.make_layer(spec, seed, tensors=tensors)
    x = synthetic.make_x(spec, T, seed)
    w_pre, w_rs = synthetic.make_gemma4_norms(spec, seed, 0)
    ei, ri = gemma4_moe_inputs(x, w_pre, w_rs, synthetic.NORM_EPS)
    ws = Workspace(layer, T)
    y, dbg = layer.forward_routed(ei, ri, workspace=ws, debug=True)
    torch.cuda.synchronize()
    ref = host_layer(spec, tensors)
    y_ref, d_ref = ref.forward(ei.cpu().numpy(), debug=True, router_in=ri.cpu().numpy())
    got = {k: v.cpu().numpy() for k, v in dbg.items()}
    t = (11 * spec.n_experts + 2 * spec.top_k - 1) // (2 * spec.top_k)
    mfma_min = max(128, min(4096, (t + 15) // 16 * 16))
    assert_parity(y.cpu().numpy(), got, y_ref, d_ref, min_identical=1.0, mfma=T >= mfma_min)
