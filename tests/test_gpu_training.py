"""GPU parity of libatlas_train_hip.so (b2_train_hip_v2) with the training oracle: every output
buffer bit-exact (both evaluate the reference's float32 loops in the same order), plus the
reference's learning check run through the trainer."""
import numpy as np
import pytest

import nets
from atlas_hip import training
from oracle import oracle

pytestmark = pytest.mark.gpu


def compare(plan, weights, inputs, labels, initial, operation="gradients"):
    x = np.asarray(inputs, np.float64)
    meta, params = training.pack(plan, x.shape[0], x.shape[1], operation)
    w = np.concatenate([np.asarray(r, np.float64) for r in weights]).astype(np.float32)
    init = np.asarray(initial, np.float32)
    lab = np.asarray(labels, np.uint64)
    got = training.run_kernel(meta, params, x.astype(np.float32), w, init, lab)
    want = oracle.train_v2(meta, params, x, w, init, lab)
    for key in want:
        assert np.array_equal(got[key].view(np.uint32), want[key].view(np.uint32)), \
            (key, np.max(np.abs(got[key].astype(np.float64) - want[key])))
    return got


@pytest.mark.parametrize("reset", ["subtract", "zero"])
@pytest.mark.parametrize("detach", [False, True])
def test_reference_vectors_bit_exact(reset, detach):
    print(f"case: training [2,2,2] reset={reset} detach={detach}", flush=True)
    plan = training.lif_training_plan([2, 2, 2], beta=0.5, reset=reset, detach_reset=detach, surrogate_slope=2)
    inputs = np.array([[[1., 0.], [0., 1.], [1., 1.], [0., 1.], [1., 0.], [1., 1.]]])
    compare(plan, [[0.8, 0.4, 0.2, 1.1], [0.9, 0.3, 0.4, 0.8]], inputs, [0], [[0.3, 1.9, 0.2, 0.1]])


@pytest.mark.parametrize("sizes,batch,time,reset,detach,window", [
    ([6, 5, 4, 3], 3, 16, "subtract", True, None),
    ([6, 5, 4, 3], 3, 16, "zero", False, 5),
    ([64, 128, 32, 10], 33, 50, "zero", False, None),
    ([64, 128, 32, 10], 33, 50, "subtract", True, 12),
    ([700, 256, 20], 6, 100, "subtract", True, None),
])
def test_random_plans_bit_exact(sizes, batch, time, reset, detach, window):
    print(f"case: training {sizes} B={batch} T={time} reset={reset} detach={detach} window={window}", flush=True)
    rng = np.random.default_rng(sum(sizes) + batch)
    plan = training.lif_training_plan(sizes, beta=0.85, reset=reset, detach_reset=detach, surrogate_slope=5,
                                      tbptt_window=window)
    weights = [list(rng.standard_normal(a * b) / np.sqrt(a) * 2.0) for a, b in zip(sizes, sizes[1:])]
    inputs = (rng.random((batch, time, sizes[0])) < 0.2).astype(float)
    labels = rng.integers(0, sizes[-1], batch)
    initial = rng.random((batch, sum(sizes[1:]))) * 0.3
    got = compare(plan, weights, inputs, labels, initial)
    assert got["spikes"].sum() > 0 and np.abs(got["gradients"]).sum() > 0


def test_hidden_learning_and_heldout():
    """test_native_training.py:88-104 through the HIP trainer: 60 Adam steps at least halve
    the loss (factor 0.6) and the held-out sequences keep the trained labels."""
    print("case: training learns the two-class task", flush=True)
    inputs = np.zeros((4, 24, 2))
    inputs[:2, :, 0] = 1
    inputs[2:, :, 1] = 1
    labels = [0, 0, 1, 1]
    plan = training.lif_training_plan([2, 2, 2], beta=0.8, learning_rate=0.04, surrogate_slope=3, logit_scale=3)
    weights = [[1.2, 0.4, 0.4, 1.2], [0.2, 0.8, 0.8, 0.2]]
    trainer = training.NativeLIFTrainer(plan, weights=weights)
    before = trainer.evaluate(inputs, labels)["loss"]
    for _ in range(60):
        trainer.step(inputs, labels)
    after = trainer.evaluate(inputs, labels)["loss"]
    assert after < before * 0.6
    assert trainer.state["weights"][0] != weights[0] and trainer.state["weights"][1] != weights[1]
    heldout = inputs.copy()
    heldout[:, ::3] = 0
    assert np.argmax(trainer.evaluate(heldout, labels)["logits"], axis=1).tolist() == labels


@pytest.mark.parametrize("reset,detach,window", [("subtract", True, None), ("zero", False, None),
                                                 ("subtract", False, 3), ("zero", True, 3)])
def test_recurrent_tied_graph_bit_exact(reset, detach, window):
    """The recurrent, tied projection graph of test_native_training_graph.py:19-35 (which the
    oracle's graph mode matches against the reference test's own float64 oracle and finite
    differences): every output buffer bit-exact, both pre planes included."""
    print(f"case: training graph reset={reset} detach={detach} window={window}", flush=True)
    plan, weights, x, labels, initial = nets.training_graph_fixture(reset, detach, window)
    got = compare(plan, weights, x, labels, initial)
    assert np.abs(got["gradients"]).sum() > 0


@pytest.mark.parametrize("stride,padding", [(1, 0), (2, 1)])
def test_conv2d_tied_graph_bit_exact_and_summed_like_the_untied_one(stride, padding):
    """A shared-kernel convolution (test_native_training_graph.py:103-136 geometry) then a dense
    readout: bit-exact with the oracle, and its tied gradients equal the untied plan's per-edge
    gradients summed per parameter id."""
    print(f"case: training conv2d stride={stride} padding={padding}", flush=True)
    conv, shape = training.conv2d_training_projection(0, 1, (2, 3, 4), 2, (2, 3), stride=stride, padding=padding)
    hidden = int(np.prod(shape))
    plan = training.lif_training_plan([24, hidden, 2], projections=[conv, training.dense_training_projection(1, 2, hidden, 2)],
                                      optimizer="sgd", learning_rate=.03, beta=.75)
    rng = np.random.default_rng(27)
    x = rng.integers(0, 2, (2, 9, 24)).astype(float)
    kernel, readout = rng.uniform(.2, .5, (2, 2, 2, 3)), rng.uniform(.1, .5, (hidden, 2))
    weights = [kernel.ravel().tolist(), readout.ravel().tolist()]
    tied = compare(plan, weights, x, [0, 1], np.zeros((2, hidden + 2)))
    untied = training.lif_training_plan([24, hidden, 2], optimizer="sgd", learning_rate=.03, beta=.75, projections=[
        dict(conv, parameter_ids=list(range(len(conv["sources"]))), parameter_count=len(conv["sources"])),
        training.dense_training_projection(1, 2, hidden, 2)])
    expanded = [[weights[0][i] for i in conv["parameter_ids"]], weights[1]]
    flat = compare(untied, expanded, x, [0, 1], np.zeros((2, hidden + 2)))
    assert np.array_equal(tied["spikes"], flat["spikes"])
    summed = np.zeros((2, conv["parameter_count"]))
    for b in range(2):
        np.add.at(summed[b], conv["parameter_ids"], flat["gradients"][b, :len(conv["sources"])].astype(np.float64))
    np.testing.assert_allclose(tied["gradients"][:, :conv["parameter_count"]], summed, rtol=1e-6, atol=1e-7)


def test_larger_random_graph_bit_exact():
    """A larger graph: 2 input projections (one sparse), a sparse tied recurrence in the hidden
    layer, a skip connection input -> output and output feedback; 33 samples, 40 ticks."""
    print("case: training random graph [50, 80, 30, 10] B=33 T=40", flush=True)
    rng = np.random.default_rng(5)
    sizes = [50, 80, 30, 10]

    def sparse(source_layer, target_layer, edges, params):
        return dict(source_layer=source_layer, target_layer=target_layer, parameter_count=params,
                    sources=rng.integers(0, sizes[source_layer], edges).tolist(),
                    targets=rng.integers(0, sizes[target_layer], edges).tolist(),
                    parameter_ids=rng.integers(0, params, edges).tolist())

    projections = [training.dense_training_projection(0, 1, 50, 80), sparse(1, 1, 900, 40),
                   training.dense_training_projection(1, 2, 80, 30), training.dense_training_projection(2, 3, 30, 10),
                   sparse(0, 3, 200, 200), sparse(3, 2, 120, 60)]
    for reset, detach, window in [("subtract", True, None), ("zero", False, 9)]:
        plan = training.lif_training_plan(sizes, projections=projections, beta=0.85, reset=reset, detach_reset=detach,
                                          surrogate_slope=5, tbptt_window=window)
        weights = [list(rng.standard_normal(p["parameter_count"]) * 0.6) for p in projections]
        x = (rng.random((33, 40, 50)) < 0.25).astype(float)
        got = compare(plan, weights, x, rng.integers(0, 10, 33), rng.random((33, 120)) * 0.3)
        assert got["spikes"].sum() > 0 and np.abs(got["gradients"]).sum() > 0


def test_dense_plan_as_projections_on_the_gpu():
    """The dense plan and the same network as dense projections give identical buffers on the GPU."""
    print("case: training dense plan as projections", flush=True)
    rng = np.random.default_rng(12)
    sizes = [64, 128, 32, 10]
    dense = training.lif_training_plan(sizes, beta=0.85, reset="zero", detach_reset=False, tbptt_window=12)
    graph = training.lif_training_plan(sizes, beta=0.85, reset="zero", detach_reset=False, tbptt_window=12,
                                       projections=[training.dense_training_projection(l, l + 1, a, b)
                                                    for l, (a, b) in enumerate(zip(sizes, sizes[1:]))])
    weights = [list(rng.standard_normal(a * b) / np.sqrt(a) * 2.0) for a, b in zip(sizes, sizes[1:])]
    x = (rng.random((17, 30, 64)) < 0.2).astype(float)
    labels, initial = rng.integers(0, 10, 17), rng.random((17, 170)) * 0.3
    a = compare(dense, weights, x, labels, initial)
    b = compare(graph, weights, x, labels, initial)
    for key in a:
        got = b[key][0] if key == "pre" else b[key]
        assert np.array_equal(got.view(np.uint32), a[key].view(np.uint32)), key
