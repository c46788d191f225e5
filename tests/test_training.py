"""The training oracle (oracle/train_oracle.c) and the training host logic, without a GPU.

The oracle restates the reference kernel's float32 loops; it is pinned by the reference's own
independent-VJP test (test_native_training.py:58-82: sizes [2,2,2], beta 0.5, slope 2, its
weights/inputs/initial vectors, both resets, detached and attached, rel 2e-5 / abs 2e-8) and by
finite differences of the frozen surrogate linearisation at larger random sizes."""
import math

import numpy as np
import pytest

import nets
import train_ref
from atlas_hip import training
from oracle import oracle


def oracle_run(plan, weights, inputs, labels, initial, operation="gradients"):
    x = np.asarray(inputs, np.float64)
    meta, params = training.pack(plan, x.shape[0], x.shape[1], operation)
    w = np.concatenate([np.asarray(r, np.float64) for r in weights])
    return oracle.train_v2(meta, params, x, w, np.asarray(initial, np.float64), np.asarray(labels))


@pytest.mark.parametrize("reset", ["subtract", "zero"])
@pytest.mark.parametrize("detach", [False, True])
def test_reference_independent_vjp_vectors(reset, detach):
    plan = training.lif_training_plan([2, 2, 2], beta=0.5, reset=reset, detach_reset=detach, surrogate_slope=2)
    weights = [[0.8, 0.4, 0.2, 1.1], [0.9, 0.3, 0.4, 0.8]]
    inputs = np.array([[[1., 0.], [0., 1.], [1., 1.], [0., 1.], [1., 0.], [1., 1.]]])
    initial = np.array([[0.3, 1.9, 0.2, 0.1]])
    out = oracle_run(plan, weights, inputs, [0], initial)
    loss, spikes, final, anchors = train_ref.forward(plan, weights, inputs, [0], initial)
    np.testing.assert_array_equal(out["spikes"], spikes)
    np.testing.assert_allclose(out["membrane"], final, rtol=0, atol=2e-7)
    assert float(out["losses"].mean()) == pytest.approx(loss, abs=2e-7)
    expected = train_ref.fd_weight_gradients(plan, weights, inputs, [0], initial)
    got = [out["gradients"][0, :4], out["gradients"][0, 4:]]
    for g, e in zip(got, expected):
        np.testing.assert_allclose(g, e, rtol=2e-5, atol=2e-8)
    epsilon = 1e-6
    for e in range(4):
        plus, minus = initial.copy(), initial.copy()
        plus[0, e] += epsilon
        minus[0, e] -= epsilon
        derivative = (train_ref.forward(plan, weights, inputs, [0], plus, anchors)[0] -
                      train_ref.forward(plan, weights, inputs, [0], minus, anchors)[0]) / (2 * epsilon)
        assert out["initial_grad"][0, e] == pytest.approx(derivative, rel=2e-5, abs=2e-8)


@pytest.mark.parametrize("reset,detach,window", [("subtract", True, None), ("zero", False, None),
                                                 ("zero", True, 5), ("subtract", False, 7)])
def test_random_plans_against_finite_differences(reset, detach, window):
    rng = np.random.default_rng(3)
    plan = training.lif_training_plan([6, 5, 4, 3], beta=0.8, reset=reset, detach_reset=detach, surrogate_slope=4,
                                      tbptt_window=window, logit_scale=3.0)
    weights = [list(rng.standard_normal(a * b) * 0.8) for a, b in zip(plan["sizes"], plan["sizes"][1:])]
    inputs = (rng.random((3, 16, 6)) < 0.4).astype(float)
    labels = [0, 2, 1]
    initial = rng.random((3, 12)) * 0.5
    out = oracle_run(plan, weights, inputs, labels, initial)
    loss, spikes, final, _ = train_ref.forward(plan, weights, inputs, labels, initial)
    np.testing.assert_array_equal(out["spikes"], spikes)
    np.testing.assert_allclose(out["membrane"], final, rtol=1e-5, atol=1e-5)
    if window is None:
        expected = train_ref.fd_weight_gradients(plan, weights, inputs, labels, initial)
        offsets = np.cumsum([0] + [len(r) for r in weights])
        total = out["gradients"].astype(np.float64).sum(axis=0)
        for l, e in enumerate(expected):
            np.testing.assert_allclose(total[offsets[l]:offsets[l + 1]], e, rtol=1e-4, atol=1e-6)
    assert spikes.sum() > 10


def test_evaluate_skips_the_backward_pass():
    plan = training.lif_training_plan([3, 4, 2], beta=0.7)
    rng = np.random.default_rng(1)
    weights = [list(rng.standard_normal(12)), list(rng.standard_normal(8))]
    inputs = (rng.random((2, 5, 3)) < 0.5).astype(float)
    out = oracle_run(plan, weights, inputs, [1, 0], np.zeros((2, 6)), operation="evaluate")
    assert not out["gradients"].any() and not out["initial_grad"].any()


def test_pack_matches_the_v2_layout():
    """gpu.rs:286-341: m[0..9] = B, T, L, I, N, E, reset_zero, detach, tbptt, backward; m[16+l] sizes;
    m[40+l] neuron offsets; m[64+l] weight offsets; params = beta, theta, slope, scale, logit_scale."""
    plan = training.lif_training_plan([7, 5, 3], beta=[0.9, 0.8], threshold=[1.0, 1.5], reset="zero",
                                      detach_reset=False, surrogate_slope=2.5, surrogate_scale=0.5, logit_scale=4.0,
                                      tbptt_window=9)
    meta, params = training.pack(plan, 4, 20, "train")
    assert list(meta[:10]) == [4, 20, 2, 7, 8, 50, 1, 0, 9, 1]
    assert list(meta[16:19]) == [7, 5, 3] and list(meta[40:43]) == [0, 5, 8] and list(meta[64:66]) == [0, 35]
    assert meta[12] == 84 and meta[13] == 7
    np.testing.assert_array_equal(params, np.float32([0.9, 0.8, 1.0, 1.5, 2.5, 0.5, 4.0]))
    meta, _ = training.pack(plan, 4, 20, "evaluate")
    assert meta[9] == 0


def test_adam_matches_the_closed_form_first_step():
    """training.rs:949-964: at step 1 the bias-corrected moments are g and g^2, so the update
    is lr * g / (|g| + eps)."""
    plan = training.lif_training_plan([2, 2, 2], learning_rate=0.1)
    trainer = training.NativeLIFTrainer(plan, weights=[[0.5] * 4, [0.25] * 4])
    grads = [[0.3, -2.0, 0.0, 1e-3], [5.0, -0.5, 0.25, -1e-4]]
    trainer._optimizer(grads)
    for l, row in enumerate(grads):
        for e, g in enumerate(row):
            start = [0.5, 0.25][l]
            assert trainer.state["weights"][l][e] == pytest.approx(start - 0.1 * g / (abs(g) + 1e-8), rel=1e-12)
    assert trainer.state["step"] == 1
    m1 = trainer.state["first_moment"][0][0]
    assert m1 == pytest.approx(0.1 * 0.3)
    assert math.isclose(trainer.state["second_moment"][0][1], 0.001 * 4.0)


@pytest.mark.parametrize("reset", ["subtract", "zero"])
@pytest.mark.parametrize("detach", [False, True])
@pytest.mark.parametrize("window", [None, 3])
def test_graph_oracle_against_the_reference_graph_test(reset, detach, window):
    """The projection-graph oracle (float32, atlas_graph_bptt's order) on the recurrent, tied
    graph of test_native_training_graph.py:19-100: the spikes equal the independent float64
    forward, the loss and final membrane agree to float32 rounding, and every weight and
    initial-state gradient equals central finite differences of the frozen-anchor
    linearisation (float32 tolerances: rel 2e-4, abs 2e-6)."""
    plan, weights, x, labels, initial = nets.training_graph_fixture(reset, detach, window)
    out = oracle_run(plan, weights, x, labels, initial)
    loss, spikes, final, _, anchors = train_ref.graph_forward(plan, weights, x, labels, initial)
    np.testing.assert_array_equal(out["spikes"], spikes)
    np.testing.assert_allclose(out["membrane"], final, rtol=0, atol=2e-6)
    assert float(out["losses"].mean()) == pytest.approx(loss, abs=2e-6)
    offsets = np.cumsum([0] + [len(w) for w in weights])
    assert np.abs(out["gradients"][:, offsets[1]:offsets[2]]).sum() > 1e-7   # the recurrence's VJP
    assert np.abs(out["gradients"][:, offsets[3]:offsets[4]]).sum() > 1e-7   # the feedback's VJP
    eps = 1e-6
    summed = out["gradients"].astype(np.float64).sum(axis=0)
    for q, w in enumerate(weights):
        for e in range(len(w)):
            plus = [list(r) for r in weights]
            minus = [list(r) for r in weights]
            plus[q][e] += eps
            minus[q][e] -= eps
            fd = (train_ref.graph_forward(plan, plus, x, labels, initial, anchors)[0] -
                  train_ref.graph_forward(plan, minus, x, labels, initial, anchors)[0]) / (2 * eps)
            assert summed[offsets[q] + e] == pytest.approx(fd, rel=2e-4, abs=2e-6), (q, e)
    for b in range(2):
        for k in range(4):
            plus, minus = initial.copy(), initial.copy()
            plus[b, k] += eps
            minus[b, k] -= eps
            fd = (train_ref.graph_forward(plan, weights, x, labels, plus, anchors)[0] -
                  train_ref.graph_forward(plan, weights, x, labels, minus, anchors)[0]) / (2 * eps)
            assert out["initial_grad"][b, k] == pytest.approx(fd, rel=2e-4, abs=2e-6), (b, k)


def test_dense_plan_as_projections_equals_the_dense_plan():
    """A dense layered plan and the same network as dense projections (target-major edges,
    source-major ids) accumulate in the same order: every output of the oracle is identical,
    and the graph's second pre plane is the membrane after the tick's inputs."""
    rng = np.random.default_rng(8)
    sizes = [6, 5, 4, 3]
    for reset, detach, window in [("subtract", True, None), ("zero", False, 5)]:
        dense = training.lif_training_plan(sizes, beta=0.8, reset=reset, detach_reset=detach, surrogate_slope=4,
                                           tbptt_window=window)
        graph = training.lif_training_plan(sizes, beta=0.8, reset=reset, detach_reset=detach, surrogate_slope=4,
                                           tbptt_window=window, projections=[
                                               training.dense_training_projection(l, l + 1, a, b)
                                               for l, (a, b) in enumerate(zip(sizes, sizes[1:]))])
        weights = [list(rng.standard_normal(a * b) * 0.8) for a, b in zip(sizes, sizes[1:])]
        x = (rng.random((3, 16, 6)) < 0.4).astype(float)
        initial = rng.random((3, 12)) * 0.5
        a = oracle_run(dense, weights, x, [0, 2, 1], initial)
        b = oracle_run(graph, weights, x, [0, 2, 1], initial)
        for key in a:
            got = b[key][0] if key == "pre" else b[key]
            assert np.array_equal(got.view(np.uint32), a[key].view(np.uint32)), key
        assert np.any(b["pre"][1] != b["pre"][0])


def test_pack_lists_the_projection_graph():
    plan, weights, x, _, _ = nets.training_graph_fixture()
    meta, params = training.pack(plan, 2, 8, "gradients")
    assert meta[10] == 4 + 4 + 4 + 4 and meta[5] == 4 + 2 + 4 + 4 and meta[12] == 84 + 4 * 16 == meta.size
    edges = meta[84:].reshape(-1, 4)
    assert edges[:4].tolist() == [[1, 0, 0, 0], [1, 1, 0, 2], [1, 0, 1, 1], [1, 1, 1, 3]]   # input -> hidden
    assert edges[4:8].tolist() == [[0, 0, 0, 4], [0, 1, 1, 4], [0, 0, 1, 5], [0, 1, 0, 5]]  # tied recurrence
    assert edges[12:].tolist() == [[0, 2, 0, 10], [0, 3, 0, 12], [0, 2, 1, 11], [0, 3, 1, 13]]  # feedback
    assert not meta[64:70].any()


def test_initial_weights_restate_the_reference_counter_stream():
    """Plan::initialize (training.rs:500-523): one splitmix64 draw per weight in bank order,
    mask * (0.25 + u) * sqrt(2 / fan_in).  Bit-level parity unpinned (no reference vectors);
    checked here for the range, the masking, the per-bank fan-in and the continuing stream."""
    plan, _, _, _, _ = nets.training_graph_fixture()
    plan["masks"][1] = [1.0, 0.0]
    w = training.initial_weights(plan)
    assert [len(r) for r in w] == [4, 2, 4, 4] and w[1][1] == 0.0
    for q, row in enumerate(w):
        scale = math.sqrt(2.0 / plan["sizes"][plan["projections"][q]["source_layer"]])
        assert all(v == 0.0 or 0.25 * scale <= v < 1.25 * scale for v in row)
    dense = training.lif_training_plan([3, 4, 2], seed=7)
    first = training.initial_weights(dense)
    assert training.initial_weights(dense) == first and len(set(first[0] + first[1])) == 20
