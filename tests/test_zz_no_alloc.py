"""b2_train_hip_v2_static (no device allocation: a static per-GPU workspace) against
b2_train_hip_v2 on the same inputs: every output buffer bit for bit, on two calls in a row,
the second with a smaller plan, and a plan beyond the workspace rejected with code 2."""
import numpy as np
import pytest

from atlas_hip import training
from atlas_hip.native import NativeError

pytestmark = pytest.mark.gpu


def _inputs(sizes, batch, time, seed):
    rng = np.random.default_rng(seed)
    plan = training.lif_training_plan(sizes, beta=0.85, reset="subtract", detach_reset=True, surrogate_slope=5)
    meta, params = training.pack(plan, batch, time, "gradients")
    w = np.concatenate([rng.standard_normal(a * b) / np.sqrt(a) * 2.0 for a, b in zip(sizes, sizes[1:])])
    x = (rng.random((batch, time, sizes[0])) < 0.2).astype(np.float32)
    labels = rng.integers(0, sizes[-1], batch).astype(np.uint64)
    initial = (rng.random((batch, sum(sizes[1:]))) * 0.3).astype(np.float32)
    return meta, params, x, w.astype(np.float32), initial, labels


def test_static_workspace_equals_the_allocating_entry_point():
    for sizes, batch, time in (([64, 128, 32, 10], 33, 50), ([6, 5, 4, 3], 3, 16)):
        print(f"case: static-workspace training {sizes} B={batch} T={time}", flush=True)
        args = _inputs(sizes, batch, time, sum(sizes) + batch)
        want = training.run_kernel(*args)
        got = training.run_kernel(*args, static_workspace=True)
        for key in want:
            assert np.array_equal(got[key].view(np.uint32), want[key].view(np.uint32)), key
        assert got["spikes"].sum() > 0 and np.abs(got["gradients"]).sum() > 0


def test_static_workspace_rejects_a_plan_beyond_its_size():
    print("case: static-workspace training beyond 64 MiB", flush=True)
    args = _inputs([700, 256, 20], 64, 100, 7)
    with pytest.raises(NativeError) as info:
        training.run_kernel(*args, static_workspace=True)
    assert info.value.code == 2 and "static workspace" in str(info.value)
