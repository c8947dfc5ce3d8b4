"""Host-side checks of the synthetic workload recipes (no GPU)."""
import numpy as np

from qwenium_amd import synthetic


def test_skew_bias_profile():
    sk = synthetic.Skew()
    E = 256
    b = sk.biases(E)
    assert b.shape == (E,)
    # exactly n_empty experts get the never-selected bias; the rest follow -a*s*ln(rank)
    assert (b == sk.empty_bias).sum() == sk.n_empty
    live = np.sort(b[b != sk.empty_bias])[::-1]
    ranks = np.arange(1, E - sk.n_empty + 1)
    np.testing.assert_allclose(live, -sk.a * sk.s * np.log(ranks), rtol=0, atol=1e-12)
    hot = sk.hot_experts(E)
    assert len(set(hot.tolist())) == 8 and b[hot[0]] == 0.0
    # a seeded permutation: hot experts are not simply 0..7
    assert sorted(hot.tolist()) != list(range(8))


def test_skew_routing_statistics_on_host():
    """The recipe's routing skew on a host-side replica (f32 numpy, small T):
    hot-8 share near one half and the forced-empty experts never selected."""
    sk = synthetic.Skew()
    H, E, K, T = 2048, 256, 8, 512
    rng = np.random.default_rng(3)
    R = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    Z = rng.standard_normal((T, H)).astype(np.float32)
    W = R + (sk.biases(E) / sk.c / np.sqrt(H)).astype(np.float32)[:, None]
    X = Z + np.float32(sk.c / np.sqrt(H))
    idx = np.argsort(-(X @ W.T), axis=1, kind="stable")[:, :K]
    cnt = np.bincount(idx.ravel(), minlength=E)
    share = cnt[sk.hot_experts(E)].sum() / (T * K)
    assert 0.4 <= share <= 0.65
    assert (cnt[sk.biases(E) == sk.empty_bias] == 0).all()


def test_stream_ids_distinct():
    ids = {synthetic.stream_id(l, s) for l in range(40) for s in synthetic.SLOTS}
    ids |= {synthetic.x_stream(b) for b in range(64)}
    ids |= {synthetic.norm_stream(l) for l in range(40)}
    assert len(ids) == 40 * len(synthetic.SLOTS) + 64 + 40
