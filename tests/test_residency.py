"""Expert-dispatch telemetry: libqmoe's MoEResidencyTracker against the
reference's own tracker (src/layers/moe_residency.cpp compiled unmodified into
oracle/_ref by oracle/Makefile), the reference's unit cases
(tests/unit/test_moe_residency.cpp:17-182) through the Python wrapper, the
batched histogram feed, and (GPU) the device dispatch histogram against the
routing's own top-k ids.

Parity bar: bit-exact (cold counts, resident sets in order, frequencies)
after every dispatch.
"""
import numpy as np
import pytest

from oracle import residency_ref
from qwenium_amd import MoEMetrics, MoEResidencyTracker, QmoeError

needs_ref = pytest.mark.skipif(not residency_ref.available(),
                               reason="oracle/_ref/libresidency_ref.so not built (no reference tree)")


def state(t):
    return (t.cold_dispatch_count(), t.resident_set(), t.frequencies(),
            [t.is_resident(e) for e in range(t.n_experts)])


# ---- the reference's unit cases ------------------------------------------------

def test_reference_cases_python_wrapper():
    t = MoEResidencyTracker(8, 3)
    assert t.cold_dispatch_count() == 0 and t.resident_set() == []
    assert MoEResidencyTracker(4, 2).frequencies() == [0, 0, 0, 0]
    with pytest.raises(RuntimeError, match=r"moe_residency: n_experts must be > 0; got 0"):
        MoEResidencyTracker(0, 1)
    with pytest.raises(RuntimeError, match=r"moe_residency: resident_k must be > 0; got 0"):
        MoEResidencyTracker(8, 0)

    t = MoEResidencyTracker(8, 2)
    for e, n in ((0, 4), (1, 3), (2, 2), (3, 1)):
        for _ in range(n):
            t.record_dispatch(e)
    assert t.resident_set() == [0, 1]
    assert [t.is_resident(e) for e in range(4)] == [True, True, False, False]

    t = MoEResidencyTracker(3, 10)
    t.record_dispatches([0, 1, 2])
    assert sorted(t.resident_set()) == [0, 1, 2]

    t = MoEResidencyTracker(8, 3)
    t.record_dispatch(4)
    assert t.resident_set() == [4]

    t = MoEResidencyTracker(8, 3)
    t.record_dispatches([0] * 5 + [1] * 4 + [2] * 3)
    before = t.cold_dispatch_count()
    t.record_dispatch(7)
    assert t.cold_dispatch_count() == before + 1
    before = t.cold_dispatch_count()
    t.record_dispatch(0)
    assert t.cold_dispatch_count() == before

    t = MoEResidencyTracker(4, 2)
    t.record_dispatch(0)
    assert t.cold_dispatch_count() == 1

    t = MoEResidencyTracker(8, 3)
    t.record_dispatches([0] * 5 + [5])
    assert t.snapshot_metrics() == MoEMetrics(t.cold_dispatch_count())

    t = MoEResidencyTracker(8, 3)
    t.record_dispatches([0] * 4 + [5])
    t.reset()
    assert t.cold_dispatch_count() == 0 and t.resident_set() == [] and t.frequencies() == [0] * 8

    t = MoEResidencyTracker(4, 1)
    t.record_dispatch(0)
    t.reset()
    t.record_dispatch(2)
    assert t.cold_dispatch_count() == 1 and t.is_resident(2)

    t = MoEResidencyTracker(8, 3)
    for bad in (-1, 8):
        with pytest.raises(QmoeError, match=rf"record_dispatch: expert_id={bad} out of range \[0, 8\)"):
            t.record_dispatch(bad)

    t = MoEResidencyTracker(4, 2)
    t.record_dispatches([0, 0, 1])
    assert t.frequencies() == [2, 1, 0, 0]


def test_cold_counts_hand_computed():
    """n=4, k=2, dispatches 0 0 1 2 2 2 1, worked by hand:
    0 cold (set empty) -> {0}; 0 warm; 1 cold -> {0,1};
    2 cold, freq 2,1,1: a tie does not displace 1 (an expert enters only when
    its frequency is strictly above the set's lowest);
    2 cold, freq 2,1,2 -> {0,2}; 2 warm, freq 2,1,3 -> [2,0]; 1 cold."""
    t = MoEResidencyTracker(4, 2)
    t.record_dispatches([0, 0, 1])
    assert t.cold_dispatch_count() == 2 and t.resident_set() == [0, 1]
    t.record_dispatch(2)
    assert t.cold_dispatch_count() == 3 and t.resident_set() == [0, 1]
    t.record_dispatch(2)
    assert t.cold_dispatch_count() == 4 and sorted(t.resident_set()) == [0, 2]
    t.record_dispatch(2)
    assert t.cold_dispatch_count() == 4 and t.resident_set() == [2, 0]
    t.record_dispatch(1)
    assert t.cold_dispatch_count() == 5 and t.frequencies() == [2, 2, 3, 0]


def test_record_rejects_bad_id_midway_keeps_prefix():
    t = MoEResidencyTracker(4, 2)
    with pytest.raises(QmoeError):
        t.record_dispatches([1, 1, 9, 2])
    assert t.frequencies() == [0, 2, 0, 0]  # dispatches before the bad id are recorded, as one by one


# ---- against the reference's own tracker ----------------------------------------

def sequences():
    rng = np.random.default_rng(7)
    out = []
    for n, k in ((1, 1), (2, 1), (3, 10), (4, 2), (8, 3), (16, 4), (64, 8), (256, 8), (256, 16), (128, 128)):
        out.append((n, k, rng.integers(0, n, 600)))                    # uniform: many ties
        out.append((n, k, rng.integers(0, min(n, 3), 300)))            # a small alphabet
        z = np.minimum(rng.zipf(1.3, 600) - 1, n - 1)                  # skewed, as routing tends to be
        out.append((n, k, rng.permutation(n)[z]))
    return out


@needs_ref
@pytest.mark.parametrize("n,k,seq", sequences())
def test_matches_reference_tracker_every_step(n, k, seq):
    ours, ref = MoEResidencyTracker(n, k), residency_ref.RefTracker(n, k)
    for i, e in enumerate(seq):
        ours.record_dispatch(int(e))
        ref.record_dispatch(int(e))
        assert state(ours) == state(ref), f"step {i} (expert {e})"
    ours.reset()
    ref.reset()
    assert state(ours) == state(ref)
    ours.record_dispatches(seq[:50])
    for e in seq[:50]:
        ref.record_dispatch(int(e))
    assert state(ours) == state(ref)


@needs_ref
def test_reference_tracker_errors_match():
    for n, k in ((0, 1), (8, 0), (8, -2), (0, 0)):
        with pytest.raises(RuntimeError) as a:
            MoEResidencyTracker(n, k)
        with pytest.raises(RuntimeError) as b:
            residency_ref.RefTracker(n, k)
        assert str(a.value) == str(b.value)
    # negative n_experts: the reference sizes its vectors from it before its own
    # check and fails there (std::length_error); both refuse, ours with the check's message
    with pytest.raises(RuntimeError, match="n_experts must be > 0; got -3"):
        MoEResidencyTracker(-3, 2)
    with pytest.raises(RuntimeError):
        residency_ref.RefTracker(-3, 2)
    ours, ref = MoEResidencyTracker(8, 3), residency_ref.RefTracker(8, 3)
    for bad in (-1, 8, 1 << 30):
        with pytest.raises(RuntimeError) as a:
            ours.record_dispatch(bad)
        with pytest.raises(RuntimeError) as b:
            ref.record_dispatch(bad)
        assert str(a.value) == str(b.value)


# ---- the batched histogram feed ----------------------------------------------------

@needs_ref
@pytest.mark.parametrize("n,k", [(16, 4), (256, 8), (64, 64)])
def test_record_counts_batches(n, k):
    """Per batch: frequencies add up, the resident set equals the reference's
    for the same frequencies (a function of the frequencies alone), and the cold
    count grows by the batch's dispatches to experts outside the set at the
    batch's start."""
    rng = np.random.default_rng(n + k)
    ours, ref = MoEResidencyTracker(n, k), residency_ref.RefTracker(n, k)
    for b in range(40):
        ids = rng.integers(0, n, int(rng.integers(0, 80)))
        counts = np.bincount(ids, minlength=n).astype(np.uint64)
        start_set = set(ours.resident_set())
        cold0 = ours.cold_dispatch_count()
        ours.record_counts(counts)
        for e in rng.permutation(ids):
            ref.record_dispatch(int(e))
        assert ours.frequencies() == ref.frequencies()
        assert ours.resident_set() == ref.resident_set(), f"batch {b}"
        assert ours.cold_dispatch_count() == cold0 + sum(int(c) for e, c in enumerate(counts) if e not in start_set)


def test_record_counts_single_dispatch_equals_record():
    rng = np.random.default_rng(3)
    a, b = MoEResidencyTracker(32, 5), MoEResidencyTracker(32, 5)
    for e in rng.integers(0, 32, 400):
        a.record_dispatch(int(e))
        one = np.zeros(32, np.uint64)
        one[e] = 1
        b.record_counts(one)
        assert state(a) == state(b)


def test_record_counts_shape_and_sign_checked():
    t = MoEResidencyTracker(8, 2)
    with pytest.raises(QmoeError, match="counts expected 8 entries, got 7"):
        t.record_counts(np.zeros(7, np.uint64))
    with pytest.raises(ValueError):
        t.record_counts(np.array([1, -1, 0, 0, 0, 0, 0, 0]))
    t.record_counts(np.zeros(8, np.uint64))
    assert state(t) == (0, [], [0] * 8, [False] * 8)


# ---- the device histogram ---------------------------------------------------------

@pytest.mark.gpu
@pytest.mark.parametrize("spec_name,Ts", [("CONFIG1", (1, 7, 300)), ("QWEN35B", (10, 1, 16, 257)),
                                          ("QWEN35B_SKEW", (10, 600))])
def test_device_histogram_equals_topk_bincount(gpu, spec_name, Ts):
    """The device histogram against a bincount of the ORACLE's top-k ids on the same
    inputs (so a routing bug that also corrupted the histogram cannot pass), the GPU's
    own top-k equal to the oracle's, and the host tracker fed from it."""
    import torch

    from oracle import pyoracle as po
    from qwenium_amd import synthetic

    spec = getattr(synthetic, spec_name)
    tensors = synthetic.make_layer_tensors(spec, 17)
    layer = synthetic.make_layer(spec, 17, tensors=tensors)
    E = spec.n_experts
    router = tensors["router"].data.cpu().numpy().reshape(E, spec.n_embd)
    counts = torch.zeros(E, dtype=torch.int64, device=gpu)
    layer.set_expert_counts(counts)
    want = np.zeros(E, np.int64)
    tracker, seq = MoEResidencyTracker(E, 8), MoEResidencyTracker(E, 8)
    for i, T in enumerate(Ts):
        x = synthetic.make_x(spec, T, 17, batch=i)
        before = counts.cpu().numpy().copy()
        _, dbg = layer.forward(x, debug=True)
        torch.cuda.synchronize()
        idx_ref, _ = po.topk_softmax(po.router_logits(router, x.cpu().numpy()), spec.top_k)
        idx = dbg["topk_idx"].cpu().numpy()
        np.testing.assert_array_equal(idx, idx_ref)
        want += np.bincount(idx_ref.reshape(-1), minlength=E)
        got = counts.cpu().numpy()
        assert np.array_equal(got, want), f"T={T}"
        tracker.record_counts(got - before)
        seq.record_dispatches(idx)
        assert tracker.frequencies() == seq.frequencies()
        assert int((got - before).sum()) == T * spec.top_k
    # detached: later forwards leave it unchanged
    layer.set_expert_counts(None)
    layer.forward(synthetic.make_x(spec, 5, 17, batch=99))
    torch.cuda.synchronize()
    assert np.array_equal(counts.cpu().numpy(), want)


@pytest.mark.gpu
def test_expert_counts_validated(gpu):
    import torch

    from qwenium_amd import synthetic

    layer = synthetic.make_layer(synthetic.CONFIG1, 1)
    for bad in (torch.zeros(15, dtype=torch.int64, device=gpu), torch.zeros(16, dtype=torch.int32, device=gpu),
                torch.zeros(16, dtype=torch.int64)):
        with pytest.raises(ValueError):
            layer.set_expert_counts(bad)
