"""Native LIF surrogate-gradient training on the MI355X (host side).

Mirrors the reference's Python trainer interface for the dense layered plan
(brian2-rust/python/brian2_rust/training.py:49-112 ``lif_training_plan``,
:114-291 ``NativeLIFTrainer``) and restates the host half of its GPU backend
(brian2-rust/src/training/gpu.rs:22-697):

* pack the v2 metadata and parameter arrays (gpu.rs:286-341, 454-462);
* call ``b2_train_hip_v2`` of libatlas_train_hip.so, which runs the forward
  pass, readout, loss and BPTT on the GPU and returns per-sample gradients;
* sum the per-sample gradients over the batch in f64, sample by sample
  (gpu.rs:607-619), apply the masks, and for ``step`` run Adam or SGD in f64
  (apply_optimizer_distributed, training.rs:924-979);
* report the batch-mean loss in f64 (gpu.rs:665).

There is no CPU fallback: without the library ``NativeUnavailable`` is raised.
"""
from __future__ import annotations

import copy
import ctypes
import math
import os
from pathlib import Path

import numpy as np

from .native import NativeError, NativeUnavailable

LIBRARY = Path(__file__).resolve().parent.parent / "libatlas_train_hip.so"
NUMERIC_PROFILE = "native-hip-forward-backward-f32-host-optimizer-f64"
_lib = None


def library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise NativeUnavailable(f"{LIBRARY} is not built (run __graft_entry__.build())")
        lib = ctypes.CDLL(str(LIBRARY))
        vp = ctypes.c_void_p
        lib.b2_train_hip_v2.argtypes = [vp] * 13 + [ctypes.c_char_p, ctypes.c_size_t]
        lib.b2_train_hip_v2.restype = ctypes.c_int
        lib.b2_train_hip_v2_static.argtypes = [vp] * 13 + [ctypes.c_char_p, ctypes.c_size_t]
        lib.b2_train_hip_v2_static.restype = ctypes.c_int
        lib.b2_train_math_v1.restype = ctypes.c_uint64
        if lib.b2_train_math_v1() != 1:
            raise NativeError(7, "training math ABI mismatch")
        _lib = lib
    return _lib


def lif_training_plan(sizes, *, backend="hip", beta=0.9, threshold=1.0, reset="subtract", detach_reset=True,
                      surrogate_slope=5.0, surrogate_scale=1.0, optimizer="adam", learning_rate=0.01, seed=1,
                      trainable=None, masks=None, logit_scale=5.0, tbptt_window=None) -> dict:
    """The dense layered plan (schema b2-lif-training-plan-v1): source-major weights,
    all thresholds before the synapses, then the reset; beta is the per-tick decay."""
    sizes = list(sizes)
    layers = len(sizes) - 1
    if not 3 <= len(sizes) <= 17 or any(type(n) is not int or not 0 < n <= 65536 for n in sizes):
        raise ValueError("training needs bounded integer input, hidden and output sizes")
    if reset not in ("subtract", "zero") or optimizer not in ("adam", "sgd"):
        raise ValueError("reset must be subtract/zero and optimizer adam/sgd")
    if tbptt_window is not None and (type(tbptt_window) is not int or tbptt_window < 1):
        raise ValueError("tbptt_window must be a positive integer")
    counts = [a * b for a, b in zip(sizes, sizes[1:])]
    return dict(schema="b2-lif-training-plan-v1", backend=backend, sizes=sizes,
                beta=[beta] * layers if isinstance(beta, (int, float)) else list(beta),
                threshold=[threshold] * layers if isinstance(threshold, (int, float)) else list(threshold),
                reset=reset, detach_reset=detach_reset,
                surrogate=dict(kind="fast_sigmoid", slope=surrogate_slope, scale=surrogate_scale),
                optimizer=dict(kind=optimizer, learning_rate=learning_rate, beta1=0.9, beta2=0.999, epsilon=1e-8),
                trainable=[True] * len(counts) if trainable is None else list(trainable),
                masks=[[1.0] * n for n in counts] if masks is None else masks,
                seed=seed, logit_scale=logit_scale, tbptt_window=tbptt_window)


def pack(plan: dict, batch: int, time: int, operation: str) -> tuple[np.ndarray, np.ndarray]:
    """v2 metadata (u64) and parameters (f32) of a dense plan (gpu.rs:286-341, 454-462)."""
    sizes = plan["sizes"]
    layers = len(sizes) - 1
    meta = np.zeros(84, np.uint64)
    neurons = sum(sizes[1:])
    edges = sum(a * b for a, b in zip(sizes, sizes[1:]))
    head = [batch, time, layers, sizes[0], neurons, edges, int(plan["reset"] == "zero"), int(plan["detach_reset"]),
            plan["tbptt_window"] or time, int(operation != "evaluate")]
    meta[:10] = head
    for l in range(layers + 1):
        meta[16 + l] = sizes[l]
    offset = 0
    for l in range(layers):
        meta[40 + l] = offset
        offset += sizes[l + 1]
    meta[40 + layers] = offset
    weights = 0
    for l in range(layers):
        meta[64 + l] = weights
        weights += sizes[l] * sizes[l + 1]
    meta[12] = len(meta)
    meta[13] = 2 * layers + 3
    params = np.array(list(plan["beta"]) + list(plan["threshold"]) +
                      [plan["surrogate"]["slope"], plan["surrogate"]["scale"], plan["logit_scale"]], np.float64)
    as32 = params.astype(np.float32)
    if not np.all(np.isfinite(as32)):
        raise ValueError("training parameter outside float32 range")
    return meta, as32


def initial_weights(plan: dict) -> list[list[float]]:
    """Gaussian weights scaled by 1/sqrt(fan_in) from the plan seed (source-major)."""
    rng = np.random.default_rng(plan["seed"])
    sizes = plan["sizes"]
    return [list(rng.standard_normal(a * b) / math.sqrt(a)) for a, b in zip(sizes, sizes[1:])]


def run_kernel(meta: np.ndarray, params: np.ndarray, x: np.ndarray, w: np.ndarray, initial: np.ndarray,
               labels: np.ndarray, *, static_workspace: bool = False) -> dict:
    """One call of b2_train_hip_v2 (or, with ``static_workspace``, of b2_train_hip_v2_static, which
    allocates no device memory); returns its output buffers as float32 arrays."""
    B, T, N, E = int(meta[0]), int(meta[1]), int(meta[4]), int(meta[5])
    C = int(meta[16 + int(meta[2])])
    arrays = dict(meta=np.ascontiguousarray(meta, np.uint64), params=np.ascontiguousarray(params, np.float32),
                  x=np.ascontiguousarray(x, np.float32), w=np.ascontiguousarray(w, np.float32),
                  initial=np.ascontiguousarray(initial, np.float32), labels=np.ascontiguousarray(labels, np.uint64))
    out = dict(pre=np.empty((B, T, N), np.float32), spikes=np.empty((B, T, N), np.float32),
               membrane=np.empty((B, N), np.float32), gradients=np.empty((B, E), np.float32),
               initial_grad=np.empty((B, N), np.float32), logits=np.empty((B, C), np.float32),
               losses=np.empty(B, np.float32))
    err = ctypes.create_string_buffer(4096)
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)  # noqa: E731
    entry = library().b2_train_hip_v2_static if static_workspace else library().b2_train_hip_v2
    rc = entry(*(ptr(arrays[k]) for k in ("meta", "params", "x", "w", "initial", "labels")),
                                   *(ptr(out[k]) for k in ("pre", "spikes", "membrane", "gradients", "initial_grad",
                                                           "logits", "losses")), err, len(err))
    if rc:
        raise NativeError(rc, err.value.decode(errors="replace"))
    return out


class NativeLIFTrainer:
    """Optimizer state plus the GPU forward/backward of a dense LIF plan.

    ``weights`` are per-layer source-major lists (reference layout); the state
    (weights, Adam moments, step) is updated by ``step`` only.
    """

    def __init__(self, plan: dict, *, weights=None):
        if plan.get("schema") != "b2-lif-training-plan-v1":
            raise ValueError("the HIP trainer runs dense layered plans (b2-lif-training-plan-v1)")
        self.plan = copy.deepcopy(plan)
        sizes = plan["sizes"]
        counts = [a * b for a, b in zip(sizes, sizes[1:])]
        weights = initial_weights(plan) if weights is None else [list(map(float, w)) for w in weights]
        if [len(w) for w in weights] != counts:
            raise ValueError("weights do not match the plan sizes")
        self.state = dict(weights=weights, first_moment=[[0.0] * n for n in counts],
                          second_moment=[[0.0] * n for n in counts], step=0)

    def step(self, inputs, labels, *, initial=None) -> dict:
        return self.execute(inputs, labels, operation="train", initial=initial)

    def gradients(self, inputs, labels, *, initial=None) -> dict:
        return self.execute(inputs, labels, operation="gradients", initial=initial)

    def evaluate(self, inputs, labels, *, initial=None) -> dict:
        return self.execute(inputs, labels, operation="evaluate", initial=initial)

    def execute(self, inputs, labels, *, operation: str = "train", initial=None) -> dict:
        if operation not in ("train", "gradients", "evaluate"):
            raise ValueError("operation must be train, gradients or evaluate")
        plan = self.plan
        x = np.asarray(inputs, np.float64)
        if x.ndim != 3 or x.shape[2] != plan["sizes"][0]:
            raise ValueError("inputs must be batch x time x input")
        batch, time, _ = x.shape
        labels = np.asarray(labels, np.int64)
        classes = plan["sizes"][-1]
        if labels.shape != (batch,) or labels.min() < 0 or labels.max() >= classes:
            raise ValueError("labels out of range")
        neurons = sum(plan["sizes"][1:])
        initial = np.zeros((batch, neurons)) if initial is None else np.asarray(initial, np.float64)
        meta, params = pack(plan, batch, time, operation)
        w = np.concatenate([np.asarray(layer, np.float64) for layer in self.state["weights"]])
        for name, values in (("inputs", x), ("weights", w), ("initial", initial)):
            if not np.all(np.isfinite(values.astype(np.float32))):
                raise ValueError(f"{name} outside float32 range")
        out = run_kernel(meta, params, x.astype(np.float32), w.astype(np.float32), initial.astype(np.float32),
                         labels.astype(np.uint64))
        offsets = np.cumsum([0] + [len(layer) for layer in self.state["weights"]])
        gradients = []
        for l, layer in enumerate(self.state["weights"]):
            acc = np.zeros(len(layer))
            for b in range(batch):          # sample by sample, as gpu.rs:607-619
                acc += out["gradients"][b, offsets[l]:offsets[l + 1]].astype(np.float64)
            gradients.append(list(acc * np.asarray(plan["masks"][l], np.float64)))
        if operation == "train":
            self._optimizer(gradients)
        loss = 0.0
        for value in out["losses"]:
            loss += float(value)
        return dict(schema="b2-lif-training-result-v1", state=copy.deepcopy(self.state), loss=loss / batch,
                    backend="hip", numeric_profile=NUMERIC_PROFILE, gradients=gradients,
                    initial_gradients=out["initial_grad"].astype(np.float64),
                    final_membrane=out["membrane"].astype(np.float64), spikes=out["spikes"].astype(np.float64),
                    logits=out["logits"].astype(np.float64), losses=out["losses"].astype(np.float64),
                    gradient_scope="tbptt-detach-boundaries" if (plan["tbptt_window"] or time) < time
                    else "full-bptt")

    def _optimizer(self, gradients) -> None:
        """Adam / SGD in f64 (training.rs:924-979)."""
        s, opt, plan = self.state, self.plan["optimizer"], self.plan
        s["step"] += 1
        for l, layer in enumerate(s["weights"]):
            if not plan["trainable"][l]:
                continue
            for e in range(len(layer)):
                if plan["masks"][l][e] == 0.0:
                    continue
                g = gradients[l][e]
                if not math.isfinite(g):
                    raise FloatingPointError("nonfinite gradient")
                if opt["kind"] == "sgd":
                    update = g
                else:
                    s["first_moment"][l][e] = opt["beta1"] * s["first_moment"][l][e] + (1.0 - opt["beta1"]) * g
                    s["second_moment"][l][e] = opt["beta2"] * s["second_moment"][l][e] + (1.0 - opt["beta2"]) * g * g
                    m = s["first_moment"][l][e] / (1.0 - math.pow(opt["beta1"], s["step"]))
                    v = s["second_moment"][l][e] / (1.0 - math.pow(opt["beta2"], s["step"]))
                    update = m / (math.sqrt(v) + opt["epsilon"])
                layer[e] -= opt["learning_rate"] * update
                if not math.isfinite(layer[e]):
                    raise FloatingPointError("nonfinite optimizer weight")


def device_from_environment() -> int:
    return int(os.environ.get("B2_TRAIN_HIP_DEVICE", "0"))
