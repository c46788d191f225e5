"""Recurrent spiking-network trainer on the MI355X (the benchmark's configuration 4).

700 Poisson input channels -> 256 recurrent current-based LIF units -> 20 leaky non-spiking
readout units, max-over-time cross-entropy, full BPTT with a fast-sigmoid surrogate, Adam.
The reference's training plans only have spike-count logits (brian2-rust/src/training/
multistate.rs:186-206), so this plan has its own schema.  The trainer object follows the shape
of the reference's ``NativeLIFTrainer`` (brian2-rust/python/brian2_rust/training.py:114-291):
``step`` trains on a batch and returns the mean loss, ``evaluate`` runs the forward pass only,
``weights`` returns the current parameters.

Everything runs in libatlas_train_hip.so (``atlas_rsnn_*``): the batched GEMMs through rocBLAS,
the tick-sequential recurrence as a hand-written fp32 MFMA kernel fused with the LIF update and
its adjoint, the readout, loss and Adam as element-wise kernels.  Weights, Adam moments and the
tapes stay resident on the device between steps.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np

from . import training
from .native import NativeError, track

DEFAULTS = {"batch": 256, "time": 100, "inputs": 700, "hidden": 256, "classes": 20,
            "tau_mem": 20e-3, "tau_syn": 5e-3, "dt": 1e-3, "threshold": 1.0, "slope": 25.0,
            "learning_rate": 1e-3, "beta1": 0.9, "beta2": 0.999, "epsilon": 1e-8}


# phases timed by atlas_rsnn_profile, in order
PHASES = ("input_gemm", "forward_ticks", "readout", "readout_adjoint", "backward_ticks", "weight_gradients", "adam")


def flops_per_sample(plan: dict) -> dict:
    """Algorithmic multiply-add FLOPs (2 per MAC) of one sample's training step, per phase."""
    T, I, H, C = plan["time"], plan["inputs"], plan["hidden"], plan["classes"]
    return {"input_gemm": 2 * T * I * H, "forward_ticks": 2 * (T - 1) * H * H, "readout": 2 * T * H * C,
            "readout_adjoint": 2 * T * C * H, "backward_ticks": 2 * (T - 1) * H * H,
            "weight_gradients": 2 * T * I * H + 2 * (T - 1) * H * H + 2 * T * H * C}


class _Spec(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_uint64), ("time", ctypes.c_uint64), ("inputs", ctypes.c_uint64),
                ("hidden", ctypes.c_uint64), ("classes", ctypes.c_uint64),
                ("alpha", ctypes.c_float), ("beta", ctypes.c_float), ("threshold", ctypes.c_float),
                ("slope", ctypes.c_float), ("learning_rate", ctypes.c_float), ("beta1", ctypes.c_float),
                ("beta2", ctypes.c_float), ("epsilon", ctypes.c_float)]


def recurrent_plan(**overrides) -> dict:
    """The configuration-4 plan: sizes, decay factors alpha = exp(-dt/tau_syn) and
    beta = exp(-dt/tau_mem), threshold, surrogate slope and Adam settings."""
    unknown = set(overrides) - set(DEFAULTS) - {"alpha", "beta"}
    if unknown:
        raise ValueError(f"unknown plan keys {sorted(unknown)}")
    plan = {**DEFAULTS, **overrides}
    plan.setdefault("alpha", math.exp(-plan["dt"] / plan["tau_syn"]))
    plan.setdefault("beta", math.exp(-plan["dt"] / plan["tau_mem"]))
    for key in ("batch", "hidden"):
        if plan[key] <= 0 or plan[key] % 16:
            raise ValueError(f"{key} must be a positive multiple of 16")
    return plan


def initial_weights(plan: dict, seed: int = 0, scale: float = 1.0) -> list[np.ndarray]:
    """Gaussian weights scaled by scale / sqrt(fan_in), float32, row-major (source, target)."""
    rng = np.random.default_rng(seed)
    shapes = [(plan["inputs"], plan["hidden"]), (plan["hidden"], plan["hidden"]), (plan["hidden"], plan["classes"])]
    return [(rng.standard_normal(s) * scale / math.sqrt(s[0])).astype(np.float32) for s in shapes]


def poisson_inputs(rng: np.random.Generator, batch: int, time: int, inputs: int, classes: int, *,
                   max_rate_hz: float = 20.0, dt: float = 1e-3):
    """Synthetic configuration-4 batch: per-channel rates uniform in [0, max_rate), Bernoulli
    spikes with probability rate * dt per (sample, tick, channel), uniform labels."""
    rates = rng.uniform(0.0, max_rate_hz, size=inputs)
    x = (rng.random((batch, time, inputs)) < rates * dt).astype(np.float32)
    return x, rng.integers(0, classes, size=batch).astype(np.uint64)


def _library():
    lib = training.library()
    if not getattr(lib, "_rsnn_bound", False):
        vp, u64 = ctypes.c_void_p, ctypes.c_uint64
        err = [ctypes.c_char_p, ctypes.c_size_t]
        lib.atlas_rsnn_create.argtypes = [ctypes.POINTER(_Spec), vp, vp, vp, ctypes.POINTER(vp), *err]
        lib.atlas_rsnn_destroy.argtypes = [vp]
        lib.atlas_rsnn_destroy.restype = None
        lib.atlas_rsnn_set_batch.argtypes = [vp, vp, vp, *err]
        lib.atlas_rsnn_step.argtypes = [vp, ctypes.c_int, u64, vp, vp, ctypes.POINTER(ctypes.c_double), *err]
        lib.atlas_rsnn_read.argtypes = [vp, ctypes.c_uint32, vp, u64, *err]
        lib.atlas_rsnn_profile.argtypes = [vp, ctypes.c_int, vp, *err]
        lib._rsnn_bound = True
    return lib


def _check(rc: int, buf, what: str) -> None:
    if rc:
        raise NativeError(f"{what} failed (code {rc}): {buf.value.decode(errors='replace')}")


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


class NativeRecurrentTrainer:
    """Resident recurrent-SNN trainer: one ``AtlasRsnn`` handle on the selected GPU."""

    def __init__(self, plan: dict, *, weights=None, seed: int = 0):
        self.plan = plan
        self.lib = _library()
        if weights is None:
            weights = initial_weights(plan, seed)
        shapes = [(plan["inputs"], plan["hidden"]), (plan["hidden"], plan["hidden"]), (plan["hidden"], plan["classes"])]
        self._initial = [np.ascontiguousarray(w, np.float32) for w in weights]
        for w, shape in zip(self._initial, shapes):
            if w.shape != shape:
                raise ValueError(f"weight shape {w.shape}, expected {shape}")
        spec = _Spec(*(plan[k] for k in ("batch", "time", "inputs", "hidden", "classes", "alpha", "beta", "threshold",
                                          "slope", "learning_rate", "beta1", "beta2", "epsilon")))
        handle = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(512)
        _check(self.lib.atlas_rsnn_create(ctypes.byref(spec), *(_ptr(w) for w in self._initial), ctypes.byref(handle),
                                          buf, 512), buf, "atlas_rsnn_create")
        self._handle = handle
        self.steps = 0
        self.device_ms = 0.0
        track(self)

    def close(self) -> None:
        if getattr(self, "_handle", None):
            self.lib.atlas_rsnn_destroy(self._handle)
            self._handle = None

    def __del__(self):
        self.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_batch(self, inputs, labels) -> None:
        p = self.plan
        x = np.ascontiguousarray(inputs, np.float32)
        if x.shape != (p["batch"], p["time"], p["inputs"]):
            raise ValueError(f"inputs shape {x.shape}, expected {(p['batch'], p['time'], p['inputs'])}")
        lab = np.ascontiguousarray(labels, np.uint64)
        if lab.shape != (p["batch"],):
            raise ValueError("one label per sample")
        buf = ctypes.create_string_buffer(512)
        _check(self.lib.atlas_rsnn_set_batch(self._handle, _ptr(x), _ptr(lab), buf, 512), buf, "atlas_rsnn_set_batch")

    def run(self, *, train: bool, repeats: int = 1) -> dict:
        """Run ``repeats`` passes over the resident batch; losses and logits of the last."""
        p = self.plan
        losses = np.empty(p["batch"], np.float32)
        logits = np.empty((p["batch"], p["classes"]), np.float32)
        ms = ctypes.c_double()
        buf = ctypes.create_string_buffer(512)
        _check(self.lib.atlas_rsnn_step(self._handle, int(train), repeats, _ptr(losses), _ptr(logits), ctypes.byref(ms),
                                        buf, 512), buf, "atlas_rsnn_step")
        if train:
            self.steps += repeats
        self.device_ms = ms.value
        return {"loss": float(np.mean(losses.astype(np.float64))), "losses": losses, "logits": logits}

    def profile(self, *, train: bool = True) -> dict:
        """One pass over the resident batch with HIP events between its phases (milliseconds)."""
        ms = np.zeros(len(PHASES), np.float64)
        buf = ctypes.create_string_buffer(512)
        _check(self.lib.atlas_rsnn_profile(self._handle, int(train), _ptr(ms), buf, 512), buf, "atlas_rsnn_profile")
        if train:
            self.steps += 1
        return dict(zip(PHASES, ms.tolist()))

    def step(self, inputs, labels) -> dict:
        self.set_batch(inputs, labels)
        return self.run(train=True)

    def evaluate(self, inputs, labels) -> dict:
        self.set_batch(inputs, labels)
        out = self.run(train=False)
        out["accuracy"] = float(np.mean(out["logits"].argmax(axis=1) == np.asarray(labels, np.int64)))
        return out

    def read(self, what: str) -> np.ndarray:
        p = self.plan
        B, T, I, H, C = (p[k] for k in ("batch", "time", "inputs", "hidden", "classes"))
        table = {"w_in": (0, (I, H)), "w_rec": (1, (H, H)), "w_out": (2, (H, C)),
                 "grad_w_in": (3, (I, H)), "grad_w_rec": (4, (H, H)), "grad_w_out": (5, (H, C)),
                 "spikes": (6, (T, B, H)), "mem_tape": (7, (T, B, H))}
        code, shape = table[what]
        out = np.empty(shape, np.float32)
        buf = ctypes.create_string_buffer(512)
        _check(self.lib.atlas_rsnn_read(self._handle, code, _ptr(out), out.size, buf, 512), buf, "atlas_rsnn_read")
        return out

    def weights(self) -> list[np.ndarray]:
        return [self.read(k) for k in ("w_in", "w_rec", "w_out")]

    def gradients(self) -> dict:
        return {k: self.read("grad_" + k) for k in ("w_in", "w_rec", "w_out")}
