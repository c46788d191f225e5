"""GPU parity of the recurrent trainer (atlas_rsnn_* in libatlas_train_hip.so) with the float64
oracle (oracle/rsnn_oracle.py).

Floating-point bar: the device computes in float32 (rocBLAS and MFMA sums in their own order),
so each tick is checked with the oracle teacher-forced by the device's own spikes (one flipped
spike near the threshold would otherwise send the two chaotic trajectories apart):

* spikes are exactly [mem > threshold] of the device's own membrane tape, and agree with the
  oracle's membrane except where it lies within 1e-5 of the threshold;
* membrane tape within 1e-5 relative to the magnitude of the terms that formed it (the oracle's
  ``mem_scale``, the recurrence over absolute values, floored at the threshold), logits within
  1e-5 of their own term magnitude (``logit_scale``) and each loss within 1e-5 of its sample's
  largest one;
* weight gradients within 1e-5 of each matrix's largest entry, against the oracle's adjoint
  evaluated on the device's own tapes: the surrogate 1/(25 |m - theta| + 1)^2 is steep enough
  that the tapes' own float32 rounding moves the gradient by ~1e-4, and that rounding is bounded
  by the membrane check above;
* Adam: the updated weights equal the float64 update of the device's own gradients within
  float32 rounding (1e-6 relative + 1e-9).
"""
import math

import numpy as np
import pytest

from atlas_hip import rsnn
from oracle import rsnn_oracle as ro

pytestmark = pytest.mark.gpu


def setup(B, T, I, H, C, *, seed=0, scale=3.0, rate=0.05, lr=0.0):
    plan = rsnn.recurrent_plan(batch=B, time=T, inputs=I, hidden=H, classes=C, learning_rate=lr)
    rng = np.random.default_rng(seed)
    x, labels = rsnn.poisson_inputs(rng, B, T, I, C, max_rate_hz=2 * rate / plan["dt"])
    weights = rsnn.initial_weights(plan, seed + 1, scale)
    return plan, x, labels, weights


def check_pass(plan, trainer, x, labels, weights, out):
    theta = plan["threshold"]
    spikes = trainer.read("spikes")
    mem = trainer.read("mem_tape")
    assert np.array_equal(spikes, (mem > theta).astype(np.float32))
    ref = ro.forward(plan, *weights, x, labels, teacher=spikes)
    scale = np.maximum(ref["mem_scale"], theta)
    d = np.abs(mem - ref["mem_tape"]) / scale
    assert d.max() <= 1e-5, (d.max(), np.median(d))
    own = ref["mem_tape"] > theta
    flips = own != (spikes > 0)
    assert np.all(np.abs(ref["mem_tape"][flips] - theta) <= 1e-5 * scale[flips])
    logit_scale = np.maximum(ref["logit_scale"], 1e-3)
    assert np.all(np.abs(out["logits"] - ref["logits"]) <= 1e-5 * logit_scale)
    loss_scale = np.maximum(logit_scale.max(axis=1), 1.0)
    assert np.all(np.abs(out["losses"] - ref["losses"]) <= 1e-5 * loss_scale)
    return spikes, dict(ref, mem_tape=mem.astype(np.float64))


# hidden sizes: 32 and 64 (one wave, masked and full), 96 (two waves, masked), 256 (the
# configuration, at batch 48 and at its full batch of 256), 272 (beyond the register-resident
# passes: one launch of the tiled kernels per tick)
@pytest.mark.parametrize("B,T,I,H,C", [(16, 20, 40, 32, 5), (32, 60, 100, 64, 10), (16, 30, 50, 96, 6),
                                       (48, 100, 700, 256, 20), (256, 100, 700, 256, 20), (16, 25, 30, 272, 5)])
def test_forward_and_gradients_match_the_oracle(B, T, I, H, C):
    print(f"case: rsnn gradients B={B} T={T} I={I} H={H} C={C}", flush=True)
    plan, x, labels, weights = setup(B, T, I, H, C)
    with rsnn.NativeRecurrentTrainer(plan, weights=weights) as trainer:
        out = trainer.step(x, labels)
        spikes, ref = check_pass(plan, trainer, x, labels, weights, out)
        assert spikes.mean() > 0.005, "case too quiet to exercise the surrogate"
        want = ro.backward(plan, *weights, x, ref)
        got = trainer.gradients()
        for key in want:
            err = np.abs(got[key] - want[key]).max()
            assert err <= 1e-5 * np.abs(want[key]).max() + 1e-12, (key, err, np.abs(want[key]).max())
        # learning rate 0: Adam is skipped and the weights stay as created
        for a, b in zip(trainer.weights(), weights):
            assert np.array_equal(a, b)


def test_real_valued_inputs():
    """Inputs that are not bfloat16 values take the float32 input projection and dW_in GEMMs
    (binary spike inputs use the split-bfloat16 ones); both meet the same bar."""
    print("case: rsnn real-valued inputs", flush=True)
    plan, x, labels, weights = setup(32, 40, 64, 128, 6)
    x = x * np.random.default_rng(9).uniform(0.5, 1.5, size=x.shape).astype(np.float32) + np.float32(1e-3)
    with rsnn.NativeRecurrentTrainer(plan, weights=weights) as trainer:
        out = trainer.step(x, labels)
        spikes, ref = check_pass(plan, trainer, x, labels, weights, out)
        assert spikes.mean() > 0.005
        want = ro.backward(plan, *weights, x, ref)
        got = trainer.gradients()
        for key in want:
            err = np.abs(got[key] - want[key]).max()
            assert err <= 1e-5 * np.abs(want[key]).max() + 1e-12, (key, err, np.abs(want[key]).max())


def test_adam_steps_match_float64_updates():
    print("case: rsnn adam", flush=True)
    plan, x, labels, weights = setup(16, 30, 40, 32, 5, lr=1e-2)
    w = [a.astype(np.float64) for a in weights]
    moments = [(np.zeros_like(a), np.zeros_like(a)) for a in w]
    with rsnn.NativeRecurrentTrainer(plan, weights=weights) as trainer:
        for step in range(1, 4):
            before = trainer.weights()
            trainer.step(x, labels)
            grads = trainer.gradients()
            after = trainer.weights()
            for k, key in enumerate(("w_in", "w_rec", "w_out")):
                # the update from this step's device weights and gradients, in float64
                new, moments[k] = ro.adam(before[k].astype(np.float64), moments[k], grads[key].astype(np.float64),
                                          step, lr=plan["learning_rate"], beta1=plan["beta1"], beta2=plan["beta2"],
                                          epsilon=plan["epsilon"])
                np.testing.assert_allclose(after[k], new, rtol=1e-6, atol=1e-9, err_msg=f"{key} step {step}")


def test_training_reduces_the_loss():
    print("case: rsnn learning", flush=True)
    plan, x, labels, weights = setup(32, 50, 60, 64, 4, lr=5e-3)
    with rsnn.NativeRecurrentTrainer(plan, weights=weights) as trainer:
        first = trainer.step(x, labels)["loss"]
        for _ in range(60):
            last = trainer.step(x, labels)["loss"]
        assert math.isfinite(last) and last < 0.7 * first, (first, last)
        assert trainer.evaluate(x, labels)["accuracy"] > 0.5


def test_repeats_equal_separate_calls():
    print("case: rsnn repeats", flush=True)
    plan, x, labels, weights = setup(16, 20, 40, 32, 5, lr=1e-3)
    with rsnn.NativeRecurrentTrainer(plan, weights=weights) as a, rsnn.NativeRecurrentTrainer(plan, weights=weights) as b:
        a.set_batch(x, labels)
        b.set_batch(x, labels)
        for _ in range(3):
            a.run(train=True)
        b.run(train=True, repeats=3)
        for u, v in zip(a.weights(), b.weights()):
            assert np.array_equal(u, v)


def test_configuration_4_shape_trains():
    """The benchmark's own shape and initialisation: B=256, T=100, 700 -> 256 -> 20."""
    print("case: rsnn configuration 4", flush=True)
    plan = rsnn.recurrent_plan()
    rng = np.random.default_rng(4)
    x, labels = rsnn.poisson_inputs(rng, 256, 100, 700, 20)
    weights = rsnn.initial_weights(plan, 5)
    with rsnn.NativeRecurrentTrainer(plan, weights=weights) as trainer:
        out = trainer.step(x, labels)
        assert np.all(np.isfinite(out["losses"]))
        check_pass(plan, trainer, x, labels, weights, out)
        for _ in range(3):
            out = trainer.step(x, labels)
        assert np.all(np.isfinite(out["losses"]))


@pytest.mark.parametrize("T", [100, 7, 5, 4, 3, 2])
def test_three_tick_passes_equal_one_tick_passes(T, monkeypatch):
    """H = 256 runs the recurrent passes three ticks per exchange (forward_tri, backward_tri); the
    one-tick passes (ATLAS_RSNN_PASSES=vec) sum each product in the same order, so tapes, adjoints,
    gradients and the Adam update are equal bit for bit, including the block boundaries of short
    runs (T not a multiple of three)."""
    print(f"case: rsnn three-tick passes against one-tick passes, B=48 T={T} H=256", flush=True)
    plan, x, labels, weights = setup(48, T, 700, 256, 20, lr=1e-3)
    runs = []
    for passes in ("vec", "tri"):
        monkeypatch.setenv("ATLAS_RSNN_PASSES", passes)
        with rsnn.NativeRecurrentTrainer(plan, weights=weights) as trainer:
            trainer.step(x, labels)
            runs.append({"mem_tape": trainer.read("mem_tape"), "spikes": trainer.read("spikes"),
                         **trainer.gradients(), "weights": trainer.weights()})
    vec, tri = runs
    # no neuron can fire before tick 3 (the membrane starts at zero and takes the current of the tick
    # before), so only the longer runs carry spikes
    assert T < 7 or vec["spikes"].mean() > 0.005
    for key in ("mem_tape", "spikes", "w_in", "w_rec", "w_out"):
        assert np.array_equal(vec[key], tri[key]), key
    for a, b in zip(vec["weights"], tri["weights"]):
        assert np.array_equal(a, b)
