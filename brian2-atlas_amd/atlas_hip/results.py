"""Result transport: ``results.bin`` (B2DMP001 v3), ``events.bin`` (B2EVT001), ``summary.json``.

Byte layout restated from the reference writer ``write_dump`` /
``write_event_monitor_dump`` (executor.rs:3147-3406; GPU writer metal.py:926-1014)
and checked against the reference's golden dump
``tests/fixtures/reference-v1/reference/results.bin``:

    "B2DMP001" u32 version=3 u32 endian=0x01020304 u64 populations u64 neurons u64 size
    per population: u64 count, steps, record_len, variables, states, spikes, last_fired,
                    has_refractory; samples per variable (tick-major, record-minor, in
                    the variable dtype); spikes (i64 tick, i64 neuron); i64 counts[count];
                    i64 last_fired; states in definition order and dtype;
                    [f64 lastspike[count], u8 not_refractory[count]]
    u64 synapses; per synapse: u64 states, u64 edges, states (dtype), u64 delivered
    f64 final_time, "B2END001"
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass

import numpy as np

from .engine import NUMPY, decode_f64

DUMP_MAGIC = b"B2DMP001"
DUMP_END = b"B2END001"
EVENT_MAGIC = b"B2EVT001"
EVENT_END = b"B2EEND01"


def _u64(value: int) -> bytes:
    return struct.pack("<Q", int(value))


def _pairs(ticks: np.ndarray, indices: np.ndarray) -> bytes:
    arr = np.empty((len(ticks), 2), "<i8")
    arr[:, 0] = ticks
    arr[:, 1] = indices
    return arr.tobytes()


def write_results(document: dict, result: dict) -> bytes:
    d = document["definition"]
    parts = []
    for pdef, pres in zip(d["populations"], result["populations"]):
        monitor = pdef["monitor"]
        ticks, idx = pres["spike_ticks"], pres["indices"]
        refr = pres["refractory"]
        head = b"".join(_u64(v) for v in (pdef["count"], pdef["steps"], len(monitor["record"]),
                                           len(monitor["variables"]), len(pdef["states"]), len(ticks),
                                           len(pres["last_spikes"]), 1 if refr is not None else 0))
        body = [head]
        for name in monitor["variables"]:
            body.append(np.ascontiguousarray(pres["trace"][name]).astype(pres["trace"][name].dtype.newbyteorder("<")).tobytes())
        body.append(_pairs(ticks, idx))
        body.append(np.asarray(pres["counts"], "<i8").tobytes())
        body.append(np.asarray(pres["last_spikes"], "<i8").tobytes())
        for symbol in pdef["states"]:
            body.append(np.asarray(pres["states"][symbol["name"]], NUMPY[symbol["dtype"]]).astype(
                np.dtype(NUMPY[symbol["dtype"]]).newbyteorder("<")).tobytes())
        if refr is not None:
            body.append(np.asarray(refr["lastspike"], "<f8").tobytes())
            body.append(np.asarray(refr["not_refractory"], np.uint8).tobytes())
        parts.append(b"".join(body))
    syn_parts = [_u64(len(d["synapses"]))]
    for sdef, sres in zip(d["synapses"], result["synapses"]):
        syn_parts.append(_u64(len(sdef["states"])) + _u64(sres["edges"]))
        for symbol in sdef["states"]:
            syn_parts.append(np.asarray(sres["states"][symbol["name"]], NUMPY[symbol["dtype"]]).astype(
                np.dtype(NUMPY[symbol["dtype"]]).newbyteorder("<")).tobytes())
        syn_parts.append(_u64(sres["events"]))
    run = document["run"]
    final = decode_f64(run["start"]) + decode_f64(run["duration"])
    tail = struct.pack("<d", final) + DUMP_END
    size = 40 + sum(len(p) for p in parts) + sum(len(p) for p in syn_parts) + len(tail)
    header = DUMP_MAGIC + struct.pack("<II", 3, 0x01020304) + _u64(len(d["populations"])) + \
        _u64(document["instance"]["neuron_count"]) + _u64(size)
    out = header + b"".join(parts) + b"".join(syn_parts) + tail
    assert len(out) == size
    return out


def write_events(document: dict, result: dict) -> bytes | None:
    d = document["definition"]
    streams = []
    for pdef, pres in zip(d["populations"], result["populations"]):
        for event in pdef["events"]:
            stream = pres["event_streams"][event]
            streams.append(_u64(len(stream["ticks"])) + _pairs(stream["ticks"], stream["indices"]))
    monitors = []
    for pdef, pres in zip(d["populations"], result["populations"]):
        symbols = {s["name"]: s for s in pdef["states"] + pdef["parameters"]}
        for monitor in pdef.get("event_monitors", []):
            rec = pres["event_monitors"][monitor["name"]]
            part = [_u64(len(rec["ticks"])), _u64(len(monitor["variables"])), _pairs(rec["ticks"], rec["indices"])]
            for name in monitor["variables"]:
                dtype = np.dtype(NUMPY[symbols[name]["dtype"]]).newbyteorder("<")
                part.append(np.asarray(rec["values"][name]).astype(dtype).tobytes())
            monitors.append(b"".join(part))
    if not streams and not monitors:
        return None
    return EVENT_MAGIC + _u64(len(streams)) + b"".join(streams) + _u64(len(monitors)) + b"".join(monitors) + EVENT_END


def summary(document: dict, result: dict, results_bytes: bytes, events_bytes: bytes | None) -> dict:
    run = document["run"]
    return {
        "dump_bytes": len(results_bytes),
        "event_dump_bytes": len(events_bytes) if events_bytes is not None else 0,
        "final_time_seconds": decode_f64(run["start"]) + decode_f64(run["duration"]),
        "neuron_count": document["instance"]["neuron_count"],
        "population_count": len(document["definition"]["populations"]),
        "schema": "b2-result-dump-v3",
        "spike_count": int(sum(len(p["spike_ticks"]) for p in result["populations"])),
        "synaptic_events": int(sum(s["events"] for s in result["synapses"])),
        "timings": {"initialization_seconds": sum(t["input_seconds"] for t in result["timings"]),
                    "simulation_and_recording_seconds": sum(t["command_seconds"] for t in result["timings"]),
                    "dump_write_seconds": result.get("dump_write_seconds", 0.0)},
        "rng_profile": result.get("rng_profile"),
        "numeric_profile": result["numeric_profile"],
        "device": result["device"],
    }


# ---------------------------------------------------------------------- reader
@dataclass
class PopulationDump:
    count: int
    steps: int
    samples: list
    spikes: np.ndarray
    counts: np.ndarray
    last_fired: np.ndarray
    states: list
    lastspike: np.ndarray | None
    not_refractory: np.ndarray | None


@dataclass
class Dump:
    populations: list
    synapses: list
    final_time: float


def read_results(data: bytes, document: dict) -> Dump:
    """Parse a B2DMP001 dump using the document for dtypes (results.py:1-140 checks)."""
    d = document["definition"]
    if data[:8] != DUMP_MAGIC or struct.unpack_from("<II", data, 8) != (3, 0x01020304):
        raise ValueError("not a B2DMP001 v3 dump")
    n_pop, _neurons, size = struct.unpack_from("<QQQ", data, 16)
    if size != len(data) or data[-8:] != DUMP_END:
        raise ValueError("truncated dump")
    o = 40
    pops = []
    for pdef in d["populations"][:n_pop]:
        count, steps, rec, nvars, nstates, nspikes, nlast, refr = struct.unpack_from("<8Q", data, o)
        o += 64
        samples = []
        dtypes = {s["name"]: s["dtype"] for s in pdef["states"] + pdef["parameters"]}
        rows = 0
        for name in pdef["monitor"]["variables"]:
            dt = np.dtype(NUMPY[dtypes[name]]).newbyteorder("<")
            nbytes = None
            # sample length is rows * rec; rows is the number of recorded ticks
            rows = min(pdef["monitor"]["window_steps"], steps)
            nbytes = rows * rec * dt.itemsize
            samples.append(np.frombuffer(data, dt, rows * rec, o).reshape(rows, rec) if rec else np.zeros((rows, 0), dt))
            o += nbytes
        spikes = np.frombuffer(data, "<i8", 2 * nspikes, o).reshape(nspikes, 2)
        o += 16 * nspikes
        counts = np.frombuffer(data, "<i8", count, o)
        o += 8 * count
        last = np.frombuffer(data, "<i8", nlast, o)
        o += 8 * nlast
        states = []
        for symbol in pdef["states"]:
            dt = np.dtype(NUMPY[symbol["dtype"]]).newbyteorder("<")
            states.append(np.frombuffer(data, dt, count, o))
            o += count * dt.itemsize
        lastspike = nr = None
        if refr:
            lastspike = np.frombuffer(data, "<f8", count, o)
            o += 8 * count
            nr = np.frombuffer(data, np.uint8, count, o)
            o += count
        pops.append(PopulationDump(count, steps, samples, spikes, counts, last, states, lastspike, nr))
    (n_syn,) = struct.unpack_from("<Q", data, o)
    o += 8
    syns = []
    for sdef in d["synapses"][:n_syn]:
        nstates, edges = struct.unpack_from("<QQ", data, o)
        o += 16
        states = []
        for symbol in sdef["states"]:
            dt = np.dtype(NUMPY[symbol["dtype"]]).newbyteorder("<")
            states.append(np.frombuffer(data, dt, edges, o))
            o += edges * dt.itemsize
        (delivered,) = struct.unpack_from("<Q", data, o)
        o += 8
        syns.append({"states": states, "edges": edges, "delivered": delivered})
    (final,) = struct.unpack_from("<d", data, o)
    return Dump(pops, syns, final)


def result_from_dump(data: bytes, document: dict) -> dict:
    """The parts of an executor result a continuation needs (final states, refractory state,
    spike streams, synapse states), read back from a B2DMP001 dump."""
    d = document["definition"]
    dump = read_results(data, document)
    populations = []
    for pdef, pop in zip(d["populations"], dump.populations):
        populations.append({
            "states": {symbol["name"]: np.array(values) for symbol, values in zip(pdef["states"], pop.states)},
            "refractory": ({"lastspike": np.array(pop.lastspike), "not_refractory": np.array(pop.not_refractory) != 0}
                           if pop.lastspike is not None else None),
            "event_streams": {"spike": {"ticks": pop.spikes[:, 0].copy(), "indices": pop.spikes[:, 1].copy()}},
        })
    synapses = [{"states": {symbol["name"]: np.array(values) for symbol, values in zip(sdef["states"], syn["states"])},
                 "events": syn["delivered"]} for sdef, syn in zip(d["synapses"], dump.synapses)]
    return {"populations": populations, "synapses": synapses}


def write_summary_json(path, summary_dict: dict) -> None:
    with open(path, "w") as handle:
        handle.write(json.dumps(summary_dict, indent=2, sort_keys=True) + "\n")
