"""Pins of the CPU oracle (oracle/liboracle.so) against independent sources:
numpy's IEEE float16, libm, exactly rounded sums (math.fsum), hand-built block
KATs, the reference's own known answers (tests/unit/test_moe.cpp:196-216,
tests/unit/test_norm.cpp:22-25) and brute force on small inputs."""
import math
import struct

import numpy as np
import pytest

from oracle import pyoracle as po

L = po.lib()


def f32(x):
    return float(np.float32(x))


def ulp_diff32(a, b):
    ia = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    ib = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


# ---- fp16 -----------------------------------------------------------------------------
def test_fp16_decode_all_patterns():
    h = np.arange(65536, dtype=np.uint16)
    got = np.array([L.qo_fp16_to_fp32(int(v)) for v in h], dtype=np.float32)
    ref = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_fp16_encode_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(20000).astype(np.float32) * (np.float32(2.0) ** rng.integers(-30, 18, 20000)).astype(
        np.float32)
    x = np.concatenate([x, np.float32([0.0, -0.0, 65504.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                                       3 * 2.0 ** -26, 6.1035156e-05, np.inf, -np.inf])])
    got = np.array([L.qo_fp32_to_fp16(float(v)) for v in x], dtype=np.uint16)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, ref)


# ---- deterministic elementary functions -------------------------------------------------
def test_exp_det_vs_libm():
    for v in np.concatenate([np.linspace(-700, 700, 4001), np.linspace(-1, 1, 2001)]):
        e, r = L.qo_exp_det(float(v)), math.exp(v)
        assert abs(e - r) <= 2 * math.ulp(r), (v, e, r)
    assert L.qo_exp_det(0.0) == 1.0
    assert L.qo_exp_det(-1000.0) == 0.0


def test_log_det_vs_libm():
    for v in np.concatenate([np.logspace(-300, 0, 3001), np.linspace(1e-6, 1, 2001)]):
        e, r = L.qo_log_det(float(v)), math.log(v)
        assert abs(e - r) <= 2 * math.ulp(r) + 1e-300, (v, e, r)
    assert L.qo_log_det(1.0) == 0.0


def test_cospi2_det_vs_libm():
    for u in np.linspace(0, 1, 20001)[:-1]:
        assert abs(L.qo_cospi2_det(float(u)) - math.cos(2 * math.pi * u)) <= 1e-15
    assert L.qo_cospi2_det(0.0) == 1.0 and L.qo_cospi2_det(0.5) == -1.0


def test_normal_generator_moments_and_determinism():
    z = po.gen_normal_f32(123, 7, 400_000)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    kurt = float(((z - z.mean()) ** 4).mean() / z.var() ** 2)
    assert abs(kurt - 3.0) < 0.05
    np.testing.assert_array_equal(z[:1000], po.gen_normal_f32(123, 7, 1000))
    assert not np.array_equal(z[:1000], po.gen_normal_f32(123, 8, 1000))


# ---- block formats ----------------------------------------------------------------------
def test_q4_0_hand_block():
    # x_j = (j % 16 - 8) * 0.5: first max-magnitude element is x_0 = -4 -> d = -4/-8 = 0.5,
    # q_j = trunc(x_j/0.5 + 8.5) = j % 16, element j+16 in the high nibble of byte j.
    x = np.array([((j % 16) - 8) * 0.5 for j in range(32)], dtype=np.float32)
    blk = po.quantize(po.TYPE_Q4_0, x)
    assert blk.size == 18
    assert struct.unpack("<e", bytes(blk[:2]))[0] == 0.5
    np.testing.assert_array_equal(blk[2:], np.array([j | (j << 4) for j in range(16)], np.uint8))
    np.testing.assert_array_equal(po.dequantize(po.TYPE_Q4_0, blk, 32), x)


def test_q4_0_nibble_layout_and_roundtrip():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(32 * 64) * 0.02).astype(np.float32)
    blk = po.quantize(po.TYPE_Q4_0, x).reshape(64, 18)
    d = blk[:, :2].copy().view(np.float16).astype(np.float32).reshape(64)
    lo = (blk[:, 2:] & 0x0F).astype(np.int32) - 8
    hi = (blk[:, 2:] >> 4).astype(np.int32) - 8
    deq = (np.concatenate([lo, hi], axis=1) * d[:, None]).reshape(-1).astype(np.float32)
    np.testing.assert_array_equal(deq, po.dequantize(po.TYPE_Q4_0, blk.reshape(-1), x.size))
    err = np.abs(deq - x).reshape(64, 32)
    # |error| <= |d|/2 except the clamped opposite extreme (q = 15), which is <= |d|
    assert np.all(err <= np.abs(d)[:, None] * 1.0000001)
    assert np.mean(err <= np.abs(d)[:, None] / 2 * 1.0000001) > 0.95


def test_q8_0_identity_block():
    x = np.array([127 - 8 * j for j in range(32)], dtype=np.float32)  # amax 127 -> d = 1
    for fn in (lambda v: po.quantize(po.TYPE_Q8_0, v), po.quantize_act):
        blk = fn(x)
        assert struct.unpack("<e", bytes(blk[:2]))[0] == 1.0
        np.testing.assert_array_equal(blk[2:].view(np.int8), x.astype(np.int8))


def test_q8_0_rounding_rules():
    # weights: quantize_row_q8_0_ref rounds half away from zero; activations:
    # the x86 SIMD quantize_row_q8_0 rounds half to even.
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1:5] = [2.5, 3.5, -2.5, -0.5]
    w = po.quantize(po.TYPE_Q8_0, x)[3:7].view(np.int8)
    a = po.quantize_act(x)[3:7].view(np.int8)
    np.testing.assert_array_equal(w, [3, 4, -3, -1])
    np.testing.assert_array_equal(a, [2, 4, -2, 0])


def test_q8_0_act_matches_numpy_restatement():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(32 * 256).astype(np.float32)
    blk = po.quantize_act(x).reshape(256, 34)
    xb = x.reshape(256, 32)
    amax = np.abs(xb).max(1)
    d16 = (amax / np.float32(127)).astype(np.float32).astype(np.float16)
    idv = (np.float32(127) / amax).astype(np.float32)
    q = np.rint(xb * idv[:, None]).astype(np.int8)
    np.testing.assert_array_equal(blk[:, :2].copy().view(np.float16).reshape(256), d16)
    np.testing.assert_array_equal(blk[:, 2:].view(np.int8), q)


@pytest.mark.parametrize("wtype", [po.TYPE_Q4_0, po.TYPE_Q8_0])
def test_vec_dot_equals_exact_dequantized_dot(wtype):
    rng = np.random.default_rng(3 + wtype)
    n = 2048
    for _ in range(20):
        w = po.quantize(wtype, (rng.standard_normal(n) * 0.02).astype(np.float32))
        xq = po.quantize_act(rng.standard_normal(n).astype(np.float32))
        wd = po.dequantize(wtype, w, n).astype(np.float64)
        xd = po.dequantize(po.TYPE_Q8_0, xq, n).astype(np.float64)
        exact = math.fsum((wd * xd).tolist())  # each product is exact in f64
        got = L.qo_vec_dot_f64(wtype, w.ctypes.data, xq.ctypes.data, n)
        assert got == exact
        assert L.qo_vec_dot(wtype, w.ctypes.data, xq.ctypes.data, n) == f32(exact)


# ---- router / top-k / sort -----------------------------------------------------------------
def test_router_logits_correctly_rounded():
    rng = np.random.default_rng(4)
    E, H, T = 16, 512, 6
    w = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((T, H)).astype(np.float32)
    got = po.router_logits(w, x)
    ref = np.array([[f32(math.fsum((w[e].astype(np.float64) * x[t]).tolist())) for e in range(E)] for t in range(T)],
                   dtype=np.float32)
    np.testing.assert_array_equal(got, ref)


def test_topk_reference_kat():
    # tests/unit/test_moe.cpp:201-215
    idx, w = po.topk_softmax(np.array([[1.0, 3.0, 0.5, 2.0, -1.0, 0.0, 4.0, 1.5]], np.float32), 2)
    assert idx.tolist() == [[6, 1]]
    e6, e1 = math.exp(4.0), math.exp(3.0)
    np.testing.assert_allclose(w[0], [e6 / (e6 + e1), e1 / (e6 + e1)], rtol=1e-6)
    np.testing.assert_allclose(w[0], [0.7310586, 0.2689414], atol=1e-6)


def test_topk_ties_lowest_index_and_brute_force():
    rng = np.random.default_rng(5)
    for trial in range(200):
        E = int(rng.integers(2, 40))
        k = int(rng.integers(1, min(E, 9) + 1))
        T = 3
        logits = rng.integers(-3, 4, size=(T, E)).astype(np.float32)  # many exact ties
        idx, w = po.topk_softmax(logits, k)
        for t in range(T):
            order = np.lexsort((np.arange(E), -logits[t]))[:k]  # desc value, asc index
            assert idx[t].tolist() == order.tolist()
            ex = np.exp(logits[t, order].astype(np.float64) - logits[t, order[0]])
            np.testing.assert_allclose(w[t], ex / ex.sum(), rtol=1e-6)


def test_sort_assignments_brute_force_and_invariants():
    rng = np.random.default_rng(6)
    for trial in range(50):
        E = int(rng.integers(1, 30))
        k = int(rng.integers(1, min(E, 6) + 1))
        T = int(rng.integers(1, 40))
        idx = np.stack([rng.permutation(E)[:k] for _ in range(T)]).astype(np.int32)
        off, rows, pos = po.sort_assignments(idx, E)
        expect_rows = [t * k + j for e in range(E) for t in range(T) for j in range(k) if idx[t, j] == e]
        assert rows.tolist() == expect_rows
        counts = np.bincount(idx.reshape(-1), minlength=E)
        np.testing.assert_array_equal(off, np.concatenate([[0], np.cumsum(counts)]))
        assert off[-1] == T * k
        np.testing.assert_array_equal(rows[pos], np.arange(T * k))
        for e in range(E):
            seg = rows[off[e]:off[e + 1]]
            assert np.all(np.diff(seg) > 0)


# ---- elementwise -----------------------------------------------------------------------------
def test_silu_and_sigmoid_vs_formula():
    rng = np.random.default_rng(7)
    for g, u in zip(rng.standard_normal(2000) * 3, rng.standard_normal(2000)):
        g, u = f32(g), f32(u)
        ref = g / (1.0 + math.exp(-g)) * u
        assert ulp_diff32(L.qo_silu_mul(g, u), ref) <= 1
        assert ulp_diff32(L.qo_sigmoid(g), 1.0 / (1.0 + math.exp(-g))) <= 1


def test_rms_norm_reference_kat():
    # tests/unit/test_norm.cpp:22-25: [3, 4] with weight [2, 0.5] -> [1.697056, 0.565685]
    for eps in (0.0, 1e-6):
        y = po.rms_norm(np.array([[3.0, 4.0]], np.float32), np.array([2.0, 0.5], np.float32), eps)
        np.testing.assert_allclose(y[0], [1.697056, 0.565685], atol=1e-4)
    y = po.rms_norm(np.array([[3.0, 4.0]], np.float32), None, 0.0)
    np.testing.assert_allclose(y[0], [0.848528, 1.131371], atol=1e-5)


def test_rms_partials_exact_on_integers():
    """Small integers: every square and sum is exact, so entry c is the integer
    sum of squares of columns 32c .. 32c+31 (a dropped, doubled or misplaced
    column fails), including the short last piece (1000 = 31 * 32 + 8)."""
    x = np.random.default_rng(3).integers(-60, 61, size=(3, 1000)).astype(np.float32)
    got = po.rms_partials(x)
    sq = (x.astype(np.int64) ** 2)
    want = np.stack([sq[:, 32 * c:32 * c + 32].sum(axis=1) for c in range(32)], axis=1).astype(np.float64)
    np.testing.assert_array_equal(got, want)


def test_rms_partials_square_rounded_to_f32():
    """Each square is rounded to f32 before the f64 sum (ggml_rms_norm's
    f64(x*x) on f32 x): the entries are the correctly rounded sums of those f32
    squares to within a few f64 ulps; summing the exact f64 squares instead
    would differ by ~1e-8 relative."""
    x = np.random.default_rng(4).standard_normal((4, 2048)).astype(np.float32)
    got = po.rms_partials(x)
    sq32 = (x * x).astype(np.float64)
    want = np.array([[math.fsum(sq32[t, 32 * c:32 * c + 32]) for c in range(64)] for t in range(4)])
    np.testing.assert_allclose(got, want, rtol=1e-15, atol=0)
    exact = np.array([[math.fsum(x[t, 32 * c:32 * c + 32].astype(np.float64) ** 2) for c in range(64)]
                      for t in range(4)])
    assert np.max(np.abs(exact - want) / want) > 1e-10  # the case separates the two


def test_rms_partials_order():
    """The order, fixed by hand-derived values where other orders round
    differently (a = 2^-54 is a quarter of an ulp of 1, 2a half of one):
    - within a run, columns in turn: a + a + a + 1 = 1 + 2^-52 (1 first gives 1;
      pairs (a+a) + (a+1) give 1 + 2^-53, a tie rounded to 1);
    - runs in adjacent pairs: runs [1, a, a, a, a, a, a, a] give
      ((1+a) + (a+a)) + ((a+a) + (a+a)) = (1 + 2^-53) + 2^-52 = 1 + 2^-52,
      while adding the runs in turn gives 1."""
    s = np.float32(2.0 ** -27)  # s * s = 2^-54 exactly in f32
    x = np.zeros((2, 32), np.float32)
    x[0, :4] = [s, s, s, 1.0]
    x[1, 0] = 1.0
    x[1, 4:32:4] = s
    got = po.rms_partials(x)
    assert got[0, 0] == 1.0 + 2.0 ** -52
    assert got[1, 0] == 1.0 + 2.0 ** -52
