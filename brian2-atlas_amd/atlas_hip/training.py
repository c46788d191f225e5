"""Native LIF surrogate-gradient training on the MI355X (host side).

Mirrors the reference's Python trainer interface for the dense layered plan and
the projection-graph plan (brian2-rust/python/brian2_rust/training.py:49-112
``lif_training_plan``, :114-291 ``NativeLIFTrainer``; training_graph.py
projection builders) and restates the host half of its GPU backend
(brian2-rust/src/training/gpu.rs:22-697):

* pack the v2 metadata and parameter arrays (gpu.rs:286-341, 454-462); a
  projection graph lists its edges after the header (gpu.rs:319-333);
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


def validate_projections(sizes, projections) -> list[int]:
    """Each projection's parameter count (training_graph.py validate_projections, training.rs:
    440-460): 1..256 projections of the six fields, a source layer (0 = the input) and a
    non-input target layer, and every source, target and parameter index inside its domain."""
    if not isinstance(projections, list) or not 1 <= len(projections) <= 256:
        raise ValueError("invalid projection count")
    counts = []
    fields = {"source_layer", "target_layer", "parameter_count", "sources", "targets", "parameter_ids"}
    for p in projections:
        if not isinstance(p, dict) or set(p) != fields:
            raise ValueError("invalid projection fields")
        source, target, count = p["source_layer"], p["target_layer"], p["parameter_count"]
        if (type(source) is not int or not 0 <= source < len(sizes) or type(target) is not int
                or not 0 < target < len(sizes)):
            raise ValueError("invalid projection layer endpoint")
        if type(count) is not int or count <= 0:
            raise ValueError("projection dimensions must be positive integers")
        edges = len(p["sources"])
        if not edges or len(p["targets"]) != edges or len(p["parameter_ids"]) != edges:
            raise ValueError("invalid projection edge/parameter shape")
        for values, limit in ((p["sources"], sizes[source]), (p["targets"], sizes[target]),
                              (p["parameter_ids"], count)):
            if any(type(v) is not int or not 0 <= v < limit for v in values):
                raise ValueError("projection index outside declared domain")
        counts.append(count)
    return counts


def dense_training_projection(source_layer: int, target_layer: int, source_count: int, target_count: int) -> dict:
    """All-to-all projection: edges target-major (each target's sources ascending), parameter ids
    source-major (source * target_count + target), one parameter per edge (training_graph.py)."""
    if min(source_count, target_count) <= 0:
        raise ValueError("projection dimensions must be positive integers")
    pairs = [(i, j) for j in range(target_count) for i in range(source_count)]
    return dict(source_layer=source_layer, target_layer=target_layer, parameter_count=source_count * target_count,
                sources=[i for i, _ in pairs], targets=[j for _, j in pairs],
                parameter_ids=[i * target_count + j for i, j in pairs])


def conv2d_training_projection(source_layer: int, target_layer: int, input_shape, out_channels: int, kernel_size,
                               *, stride: int = 1, padding: int = 0):
    """Shared-kernel 2-D cross-correlation (OIHW kernel, CHW layers, zero padding): one edge per
    (output position, in-bounds kernel tap), ordered by output channel, row, column, then input
    channel and tap; every use of a coefficient shares its parameter id (training_graph.py).
    Returns (projection, output CHW shape)."""
    channels, height, width = input_shape
    kh, kw = (kernel_size, kernel_size) if type(kernel_size) is int else tuple(kernel_size)
    if min(channels, height, width, out_channels, kh, kw, stride) <= 0 or padding < 0:
        raise ValueError("projection dimensions must be positive integers")
    oh, ow = (height + 2 * padding - kh) // stride + 1, (width + 2 * padding - kw) // stride + 1
    if oh <= 0 or ow <= 0:
        raise ValueError("projection dimensions must be positive integers")
    sources, targets, ids = [], [], []
    for oc in range(out_channels):
        for oy in range(oh):
            for ox in range(ow):
                for ic in range(channels):
                    for ky in range(kh):
                        for kx in range(kw):
                            iy, ix = oy * stride + ky - padding, ox * stride + kx - padding
                            if 0 <= iy < height and 0 <= ix < width:
                                sources.append((ic * height + iy) * width + ix)
                                targets.append((oc * oh + oy) * ow + ox)
                                ids.append(((oc * channels + ic) * kh + ky) * kw + kx)
    if not sources:
        raise ValueError("convolution has no input edges")
    return (dict(source_layer=source_layer, target_layer=target_layer, parameter_count=out_channels * channels * kh * kw,
                 sources=sources, targets=targets, parameter_ids=ids), (out_channels, oh, ow))


def lif_training_plan(sizes, *, backend="hip", beta=0.9, threshold=1.0, reset="subtract", detach_reset=True,
                      surrogate_slope=5.0, surrogate_scale=1.0, optimizer="adam", learning_rate=0.01, seed=1,
                      trainable=None, masks=None, logit_scale=5.0, tbptt_window=None, projections=None) -> dict:
    """The dense layered plan (schema b2-lif-training-plan-v1): source-major weights,
    all thresholds before the synapses, then the reset; beta is the per-tick decay.  With
    ``projections`` the plan is b2-lif-training-plan-v2: an ordered edge list per projection
    whose parameter ids index its own weight bank (tied ids share a weight and its optimizer
    slot); masks, trainable and weights are then per bank."""
    sizes = list(sizes)
    layers = len(sizes) - 1
    if not 3 <= len(sizes) <= 17 or any(type(n) is not int or not 0 < n <= 65536 for n in sizes):
        raise ValueError("training needs bounded integer input, hidden and output sizes")
    if reset not in ("subtract", "zero") or optimizer not in ("adam", "sgd"):
        raise ValueError("reset must be subtract/zero and optimizer adam/sgd")
    if tbptt_window is not None and (type(tbptt_window) is not int or tbptt_window < 1):
        raise ValueError("tbptt_window must be a positive integer")
    counts = ([a * b for a, b in zip(sizes, sizes[1:])] if projections is None
              else validate_projections(sizes, projections))
    plan = dict(schema="b2-lif-training-plan-v1", backend=backend, sizes=sizes,
                beta=[beta] * layers if isinstance(beta, (int, float)) else list(beta),
                threshold=[threshold] * layers if isinstance(threshold, (int, float)) else list(threshold),
                reset=reset, detach_reset=detach_reset,
                surrogate=dict(kind="fast_sigmoid", slope=surrogate_slope, scale=surrogate_scale),
                optimizer=dict(kind=optimizer, learning_rate=learning_rate, beta1=0.9, beta2=0.999, epsilon=1e-8),
                trainable=[True] * len(counts) if trainable is None else list(trainable),
                masks=[[1.0] * n for n in counts] if masks is None else masks,
                seed=seed, logit_scale=logit_scale, tbptt_window=tbptt_window)
    if projections is not None:
        plan.update(schema="b2-lif-training-plan-v2", projections=copy.deepcopy(projections))
    return plan


def parameter_counts(plan: dict) -> list[int]:
    """Weights per bank: one bank per layer (v1) or per projection (v2)."""
    if plan.get("projections") is not None:
        return [p["parameter_count"] for p in plan["projections"]]
    sizes = plan["sizes"]
    return [a * b for a, b in zip(sizes, sizes[1:])]


def pack(plan: dict, batch: int, time: int, operation: str) -> tuple[np.ndarray, np.ndarray]:
    """v2 metadata (u64) and parameters (f32) of a plan (gpu.rs:286-341, 454-462): for a
    projection graph, meta[10] edges follow the header as (input, source, target, parameter),
    sources and targets as network neuron indices (input channels for input edges) and the
    parameter as its bank offset plus its id."""
    sizes = plan["sizes"]
    layers = len(sizes) - 1
    meta = np.zeros(84, np.uint64)
    neurons = sum(sizes[1:])
    edges = sum(parameter_counts(plan))
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
    projections = plan.get("projections")
    if projections is None:
        weights = 0
        for l in range(layers):
            meta[64 + l] = weights
            weights += sizes[l] * sizes[l + 1]
    else:
        bank = np.cumsum([0] + [p["parameter_count"] for p in projections])
        rows = []
        for q, p in enumerate(projections):
            src = np.asarray(p["sources"], np.uint64)
            if p["source_layer"]:
                src = src + meta[39 + p["source_layer"]]
            rows.append(np.stack([np.full(src.size, int(p["source_layer"] == 0), np.uint64), src,
                                  np.asarray(p["targets"], np.uint64) + meta[39 + p["target_layer"]],
                                  np.asarray(p["parameter_ids"], np.uint64) + np.uint64(bank[q])], axis=1))
        graph = np.concatenate(rows).reshape(-1)
        meta[10] = graph.size // 4
        meta = np.concatenate([meta, graph])
    meta[12] = len(meta)
    meta[13] = 2 * layers + 3
    params = np.array(list(plan["beta"]) + list(plan["threshold"]) +
                      [plan["surrogate"]["slope"], plan["surrogate"]["scale"], plan["logit_scale"]], np.float64)
    as32 = params.astype(np.float32)
    if not np.all(np.isfinite(as32)):
        raise ValueError("training parameter outside float32 range")
    return meta, as32


def initial_weights(plan: dict) -> list[list[float]]:
    """The reference's initial weights (Plan::initialize, training.rs:500-523): a splitmix64
    counter stream from the plan seed, one draw per weight of every bank in order,
    mask * (0.25 + u) * sqrt(2 / fan_in), fan_in the size of the bank's source layer."""
    mask64 = (1 << 64) - 1
    state = int(plan["seed"]) & mask64
    sizes = plan["sizes"]
    projections = plan.get("projections")
    weights = []
    for bank, mask in enumerate(plan["masks"]):
        source = bank if projections is None else projections[bank]["source_layer"]
        scale = math.sqrt(2.0 / sizes[source])
        values = []
        for active in mask:
            state = (state + 0x9E3779B97F4A7C15) & mask64
            z = state
            z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask64
            z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask64
            z ^= z >> 31
            values.append(float(active) * (0.25 + (z >> 11) / 9007199254740992.0) * scale)
        weights.append(values)
    return weights


def run_kernel(meta: np.ndarray, params: np.ndarray, x: np.ndarray, w: np.ndarray, initial: np.ndarray,
               labels: np.ndarray, *, static_workspace: bool = False) -> dict:
    """One call of b2_train_hip_v2 (or, with ``static_workspace``, of b2_train_hip_v2_static, which
    allocates no device memory); returns its output buffers as float32 arrays."""
    B, T, N, E = int(meta[0]), int(meta[1]), int(meta[4]), int(meta[5])
    C = int(meta[16 + int(meta[2])])
    arrays = dict(meta=np.ascontiguousarray(meta, np.uint64), params=np.ascontiguousarray(params, np.float32),
                  x=np.ascontiguousarray(x, np.float32), w=np.ascontiguousarray(w, np.float32),
                  initial=np.ascontiguousarray(initial, np.float32), labels=np.ascontiguousarray(labels, np.uint64))
    # a projection graph's pre tape has two planes: u, then the membrane after the tick's edges
    pre_shape = (2, B, T, N) if int(meta[10]) else (B, T, N)
    out = dict(pre=np.empty(pre_shape, np.float32), spikes=np.empty((B, T, N), np.float32),
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
    """Optimizer state plus the GPU forward/backward of a dense or projection-graph LIF plan.

    ``weights`` are per-bank lists (reference layout: per layer source-major, or per projection
    by parameter id); the state (weights, Adam moments, step) is updated by ``step`` only.
    """

    def __init__(self, plan: dict, *, weights=None):
        if plan.get("schema") not in ("b2-lif-training-plan-v1", "b2-lif-training-plan-v2"):
            raise ValueError("the HIP trainer runs dense layered and projection-graph LIF plans (v1, v2)")
        self.plan = copy.deepcopy(plan)
        counts = parameter_counts(plan)
        weights = initial_weights(plan) if weights is None else [list(map(float, w)) for w in weights]
        if [len(w) for w in weights] != counts or [len(m) for m in plan["masks"]] != counts:
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
