"""GPU parity of libatlas_train_hip.so (b2_train_hip_v2) with the training oracle: every output
buffer bit-exact (both evaluate the reference's float32 loops in the same order), plus the
reference's learning check run through the trainer."""
import numpy as np
import pytest

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
