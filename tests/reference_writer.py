"""Restatement of the reference's GPU result writer, for the executor-contract tests.

``write_gpu_results`` makes every read that ``_write_gpu_results``
(brian2-rust/python/brian2_rust/metal.py:926-1014) makes on an executor result
dictionary — profile checks, per-population arrays, per-synapse states and event
counts, event streams and event monitors, the ``timings`` list — and writes the
same three files.  It is test code: the product writes its files with
``atlas_hip.results``; this module shows that a ``HipExecutor.run()`` result
satisfies the reference consumer the INTEGRATION binding hands it to.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np

from atlas_hip.engine import decode_f64
from atlas_hip.executor import has_random

DTYPES = {"f32": "<f4", "f64": "<f8", "i32": "<i4", "i64": "<i8", "u32": "<u4", "u64": "<u8", "bool": "u1"}
REFERENCE_GPU_RNG_PROFILE = "b2-counter-f32-u24-v0"   # metal_random.py:9


class ConsumerRejected(ValueError):
    """The reference writer's PlanValidationError."""


def write_gpu_results(model: dict, result: dict, directory, *, engine: str, numeric_profile: str,
                      rng_profile: str | None = REFERENCE_GPU_RNG_PROFILE) -> dict:
    """Write results.bin / events.bin / summary.json from ``result`` as metal.py:926-1014 does.
    ``rng_profile`` is the profile the consumer demands of models with random draws."""
    if result.get("numeric_profile") != numeric_profile:
        raise ConsumerRejected(f"{engine} transport requires its own float32 result")
    if result.get("rng_profile") != (rng_profile if has_random(model["definition"]) else None):
        raise ConsumerRejected("GPU result RNG profile does not match model")
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=False)
    final = decode_f64(model["run"]["start"]) + decode_f64(model["run"]["duration"])
    d = model["definition"]
    out = bytearray(struct.pack("<8sIIQQQ", b"B2DMP001", 3, 0x01020304, len(result["populations"]),
                                model["instance"]["neuron_count"], 0))
    for pdef, values in zip(d["populations"], result["populations"], strict=True):
        monitor = pdef["monitor"]
        out += struct.pack("<8Q", pdef["count"], pdef["steps"], len(monitor["record"]), len(monitor["variables"]),
                           len(pdef["states"]), len(values["indices"]), len(values["last_spikes"]),
                           int(values["refractory"] is not None))
        symbols = {s["name"]: s for s in pdef["states"] + pdef["parameters"] + pdef.get("linked_variables", [])}
        for name in monitor["variables"]:
            out += np.asarray(values["trace"][name], DTYPES[symbols[name]["dtype"]]).tobytes()
        out += np.column_stack((values["spike_ticks"], values["indices"])).astype("<i8").tobytes()
        out += np.asarray(values["counts"], "<i8").tobytes()
        out += np.asarray(values["last_spikes"], "<i8").tobytes()
        for state in pdef["states"]:
            out += np.asarray(values["states"][state["name"]], DTYPES[state["dtype"]]).tobytes()
        if values["refractory"] is not None:
            out += np.asarray(values["refractory"]["lastspike"], "<f8").tobytes()
            out += np.asarray(values["refractory"]["not_refractory"], "u1").tobytes()
    out += struct.pack("<Q", len(d["synapses"]))
    for q, sdef in enumerate(d["synapses"]):
        values = result["synapses"][q]
        inst = model["instance"]["synapses"][q]
        edges = inst.get("topology", {}).get("edge_count", len(inst["source"]))
        out += struct.pack("<2Q", len(sdef["states"]), edges)
        for state in sdef["states"]:
            out += np.asarray(values["states"][state["name"]], DTYPES[state["dtype"]]).tobytes()
        out += struct.pack("<Q", values["events"])
    out += struct.pack("<d8s", final, b"B2END001")
    struct.pack_into("<Q", out, 32, len(out))
    (directory / "results.bin").write_bytes(bytes(out))
    event_bytes = 0
    if any(pop.get("event_streams") for pop in result["populations"]):
        streams = [(p, event) for p, pdef in enumerate(d["populations"]) for event in pdef["events"]]
        ev = bytearray(b"B2EVT001" + struct.pack("<Q", len(streams)))
        for p, event in streams:
            values = result["populations"][p]["event_streams"][event]
            ev += struct.pack("<Q", len(values["ticks"]))
            ev += np.column_stack((values["ticks"], values["indices"])).astype("<i8").tobytes()
        monitors = [(p, m) for p, pdef in enumerate(d["populations"]) for m in pdef.get("event_monitors", [])]
        ev += struct.pack("<Q", len(monitors))
        for p, monitor in monitors:
            values = result["populations"][p]["event_monitors"][monitor["name"]]
            ev += struct.pack("<2Q", len(values["ticks"]), len(monitor["variables"]))
            ev += np.column_stack((values["ticks"], values["indices"])).astype("<i8").tobytes()
            pdef = d["populations"][p]
            symbols = {s["name"]: s for s in pdef["states"] + pdef["parameters"] + pdef.get("linked_variables", [])}
            for name in monitor["variables"]:
                ev += np.asarray(values["values"][name], DTYPES[symbols[name]["dtype"]]).tobytes()
        ev += b"B2EEND01"
        (directory / "events.bin").write_bytes(bytes(ev))
        event_bytes = len(ev)
    summary = {"schema": "b2-result-dump-v3", "engine": engine,
               "initializations": result.get("initializations", []),
               "initialization_seconds": result.get("initialization_seconds", 0.0),
               "rng_profile": result.get("rng_profile"), "numeric_profile": numeric_profile,
               "device": result["device"], "event_dump_bytes": event_bytes, "plan_sha256": result["plan_sha256"],
               "dump_bytes": len(out), "population_count": len(result["populations"]),
               "neuron_count": model["instance"]["neuron_count"],
               "spike_count": sum(len(p["indices"]) for p in result["populations"]),
               "synaptic_events": sum(s["events"] for s in result.get("synapses", [])),
               "final_time_seconds": final,
               "timings": {"initialization_seconds": sum(t["input_seconds"] for t in result["timings"]),
                           "simulation_and_recording_seconds": sum(t["command_seconds"] for t in result["timings"]),
                           "dump_write_seconds": 0.0},
               f"{engine}_timings": result["timings"], "run_seconds": result["run_seconds"],
               "compile_seconds": result["compile_seconds"]}
    (directory / "summary.json").write_text(json.dumps(summary, indent=2) + "\n")
    return summary
