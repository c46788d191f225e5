"""ctypes wrapper of the CPU oracle (``liboracle.so``).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s CPU-baseline leg, never by the product package.

``run(model)`` executes an AtlasIR document with the C restatement of the
reference ``b2-runner`` executor and returns the ``results.bin`` / ``events.bin``
bytes it would write (executor.rs:4774-4824), plus the counters that
``summary.json`` carries.
"""
from __future__ import annotations

import ctypes
import subprocess
from dataclasses import dataclass
from pathlib import Path

from . import ir_compile

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"


class _Output(ctypes.Structure):
    _fields_ = [("results", ctypes.POINTER(ctypes.c_uint8)), ("results_len", ctypes.c_size_t),
                ("events", ctypes.POINTER(ctypes.c_uint8)), ("events_len", ctypes.c_size_t),
                ("has_events", ctypes.c_int),
                ("spike_count", ctypes.c_uint64), ("synaptic_events", ctypes.c_uint64),
                ("ticks_run", ctypes.c_uint64), ("sim_seconds", ctypes.c_double)]


@dataclass
class OracleResult:
    results: bytes
    events: bytes | None
    spike_count: int
    synaptic_events: int
    ticks_run: int
    sim_seconds: float


class OracleError(RuntimeError):
    pass


def build(force: bool = False) -> Path:
    """Compile the C oracle with the committed Makefile recipe."""
    newest = max((HERE / name).stat().st_mtime for name in ("atlas_oracle.c", "train_oracle.c"))
    if force or not LIBRARY.exists() or LIBRARY.stat().st_mtime < newest:
        subprocess.run(["make", "-s", "-B" if force else "-s", "-C", str(HERE)], check=True)
    return LIBRARY


_lib = None


def library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        lib = ctypes.CDLL(str(LIBRARY))
        lib.oracle_run.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.c_int64, ctypes.POINTER(_Output),
                                   ctypes.c_char_p, ctypes.c_size_t]
        lib.oracle_run.restype = ctypes.c_int
        lib.oracle_free.argtypes = [ctypes.POINTER(_Output)]
        lib.oracle_fixed_indegree.argtypes = [ctypes.c_uint64] * 4 + [ctypes.c_void_p] * 2
        lib.oracle_fixed_total.argtypes = [ctypes.c_uint64] * 4 + [ctypes.c_void_p] * 2
        lib.oracle_uniform.argtypes = [ctypes.c_uint64] * 3 + [ctypes.c_double] * 2 + [ctypes.c_void_p]
        lib.oracle_counter_uniform.argtypes = [ctypes.c_uint64] * 4
        lib.oracle_counter_uniform.restype = ctypes.c_double
        lib.oracle_set_shared_math.argtypes = [ctypes.c_int]
        lib.oracle_set_shared_math.restype = None
        lib.oracle_math.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_void_p]
        lib.oracle_math.restype = None
        lib.oracle_initializer.argtypes = ([ctypes.c_int] + [ctypes.c_uint64] * 3 + [ctypes.c_double] * 4
                                           + [ctypes.c_int] * 2 + [ctypes.c_void_p])
        lib.oracle_initializer.restype = ctypes.c_int
        lib.oracle_counter_normal.argtypes = [ctypes.c_uint64] * 4 + [ctypes.c_int]
        lib.oracle_counter_normal.restype = ctypes.c_double
        u64, f64, i32 = ctypes.c_uint64, ctypes.c_double, ctypes.c_int
        for name, args in (("oracle_counter_uniform_draw", [u64] * 5),
                           ("oracle_counter_binomial", [u64] * 5 + [f64, i32, i32]),
                           ("oracle_binomial_search", [f64, u64, f64, i32]),
                           ("oracle_counter_poisson", [u64] * 4 + [f64, i32]),
                           ("oracle_ptrs_trial", [f64, f64, f64, i32])):
            getattr(lib, name).argtypes = args
            getattr(lib, name).restype = f64
        _lib = lib
    return _lib


def run_blob(blob: bytes, max_ticks: int = 0, shared_math: bool = False) -> OracleResult:
    lib = library()
    out = _Output()
    err = ctypes.create_string_buffer(1024)
    lib.oracle_set_shared_math(1 if shared_math else 0)
    try:
        rc = lib.oracle_run(blob, len(blob), max_ticks, ctypes.byref(out), err, len(err))
    finally:
        lib.oracle_set_shared_math(0)
    if rc != 0:
        raise OracleError(err.value.decode())
    try:
        results = ctypes.string_at(out.results, out.results_len)
        events = ctypes.string_at(out.events, out.events_len) if out.has_events else None
        return OracleResult(results, events, out.spike_count, out.synaptic_events, out.ticks_run, out.sim_seconds)
    finally:
        lib.oracle_free(ctypes.byref(out))


def run(model, *, max_ticks: int = 0, lift_recording_budget: bool = False, shared_math: bool = False) -> OracleResult:
    """Run an AtlasIR document (path or dict) through the oracle.

    ``shared_math`` evaluates exp / expm1 / exprel of per-neuron and per-event
    statements with the engines' shared implementation (atlas_math.h) instead of
    the host libm; the GPU engine always uses the shared implementation there.
    """
    return run_blob(ir_compile.compile_model(model, lift_recording_budget=lift_recording_budget), max_ticks,
                    shared_math)


def math(which: str, x):
    """(shared, libm) values of exp / expm1 / exprel / log over an f64 array."""
    import numpy as np
    x = np.ascontiguousarray(x, np.float64)
    shared, libm = np.empty_like(x), np.empty_like(x)
    library().oracle_math({"exp": 0, "expm1": 1, "exprel": 2, "log": 3}[which], x.ctypes.data, x.size,
                          shared.ctypes.data, libm.ctypes.data)
    return shared, libm


def fixed_indegree(n_src: int, n_tgt: int, indegree: int, seed: int):
    import numpy as np
    src = np.zeros(n_tgt * indegree, np.uint32)
    tgt = np.zeros(n_tgt * indegree, np.uint32)
    if library().oracle_fixed_indegree(n_src, n_tgt, indegree, seed, src.ctypes.data, tgt.ctypes.data):
        raise OracleError("invalid fixed-indegree topology specification")
    return src, tgt


def fixed_total(n_src: int, n_tgt: int, edges: int, seed: int):
    import numpy as np
    src = np.zeros(edges, np.uint32)
    tgt = np.zeros(edges, np.uint32)
    if library().oracle_fixed_total(n_src, n_tgt, edges, seed, src.ctypes.data, tgt.ctypes.data):
        raise OracleError("invalid fixed-total topology specification")
    return src, tgt


def uniform(count: int, seed: int, stream: int, minimum: float, maximum: float):
    import numpy as np
    out = np.zeros(count, np.float64)
    if library().oracle_uniform(count, seed, stream, minimum, maximum, out.ctypes.data):
        raise OracleError("invalid uniform initializer")
    return out


def counter_uniform(seed: int, stream: int, tick: int, index: int) -> float:
    return library().oracle_counter_uniform(seed, stream, tick, index)


def counter_normal(seed: int, stream: int, tick: int, index: int, *, shared: bool = False) -> float:
    """counter_normal (executor.rs:206-221); ``shared`` takes the logarithm from atlas_math.h."""
    return library().oracle_counter_normal(seed, stream, tick, index, 1 if shared else 0)


def counter_uniform_draw(seed: int, stream: int, tick: int, index: int, draw: int) -> float:
    return library().oracle_counter_uniform_draw(seed, stream, tick, index, draw)


def counter_binomial(seed: int, stream: int, tick: int, index: int, n: int, p: float, approximate: bool, *,
                     shared: bool = False) -> float:
    """counter_binomial (executor.rs:224-268) as vector code evaluates it."""
    return library().oracle_counter_binomial(seed, stream, tick, index, n, p, int(approximate), int(shared))


def binomial_search(u: float, n: int, probability: float, *, shared: bool = False) -> float:
    """One inversion search of counter_binomial on the uniform u: x, or -1 past the restart bound."""
    return library().oracle_binomial_search(u, n, probability, int(shared))


def counter_poisson(seed: int, stream: int, tick: int, index: int, lam: float, *, shared: bool = False) -> float:
    """counter_poisson (executor.rs:290-323) as vector code evaluates it."""
    return library().oracle_counter_poisson(seed, stream, tick, index, lam, int(shared))


def ptrs_trial(u: float, v: float, lam: float, *, shared: bool = False) -> float:
    """One PTRS trial of counter_poisson on the uniforms (u, v): the candidate, or -1 if rejected."""
    return library().oracle_ptrs_trial(u, v, lam, int(shared))


def clipped_normal(count: int, seed: int, stream: int, mean: float, std: float,
                   minimum: float | None = None, maximum: float | None = None):
    """materialize_clipped_normal (large_topology.rs:95-127) over edges 0..count-1."""
    import numpy as np
    out = np.zeros(count, np.float64)
    if library().oracle_initializer(1, count, seed, stream, 0.0 if minimum is None else minimum,
                                    0.0 if maximum is None else maximum, mean, std,
                                    minimum is not None, maximum is not None, out.ctypes.data):
        raise OracleError("clipped-normal initializer failed")
    return out


def train_v2(meta, params, x, w, initial, labels) -> dict:
    """The training oracle (train_oracle.c) on the v2 buffers; returns its outputs."""
    import numpy as np
    lib = library()
    fn = lib.oracle_train_v2
    fn.argtypes = [ctypes.c_void_p] * 13
    fn.restype = ctypes.c_int
    meta = np.ascontiguousarray(meta, np.uint64)
    B, T, N, E = int(meta[0]), int(meta[1]), int(meta[4]), int(meta[5])
    C = int(meta[16 + int(meta[2])])
    ins = [np.ascontiguousarray(a, d) for a, d in ((meta, np.uint64), (params, np.float32), (x, np.float32),
                                                    (w, np.float32), (initial, np.float32), (labels, np.uint64))]
    # a projection graph's pre tape has two planes: u, then the membrane after the tick's edges
    pre_shape = (2, B, T, N) if int(meta[10]) else (B, T, N)
    out = dict(pre=np.empty(pre_shape, np.float32), spikes=np.empty((B, T, N), np.float32),
               membrane=np.empty((B, N), np.float32), gradients=np.empty((B, E), np.float32),
               initial_grad=np.empty((B, N), np.float32), logits=np.empty((B, C), np.float32),
               losses=np.empty(B, np.float32))
    rc = fn(*(a.ctypes.data for a in ins), *(out[k].ctypes.data for k in ("pre", "spikes", "membrane", "gradients",
                                                                          "initial_grad", "logits", "losses")))
    if rc:
        raise OracleError("training oracle failed")
    return out
