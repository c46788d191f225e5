"""Continuation documents: the AtlasIR of the next run segment from a finished run.

AtlasIR.md section 6: a segmented run equals the continuous run when the instance carries the
final states, refractory state, synapse states and the pending delayed events over the
boundary.  The reference Device builds that instance from a run's results
(brian2_rust/device.py:2200-2370, ``_next_pending_events`` and ``_inject_pending_events``);
``continuation`` restates it for documents run by HipExecutor (or the oracle):

* populations start from the run's final states, ``lastspike`` and ``not_refractory``;
* a SpikeGeneratorGroup keeps the part of its schedule inside the new run;
* synapses start from their final states; each pathway's pending events are the arrivals at
  or after the boundary of spikes emitted in the run: (spike tick + delay, source) for a
  uniform delay, (spike tick + the edge's delay, edge) per edge otherwise (device.py:2330-2362),
  ordered by delivery tick;
* the run starts where the previous one ended.

The event streams must cover the last ``max delay`` ticks of the run (recording window).
"""
from __future__ import annotations

import copy
import struct

import numpy as np

from . import protocol
from .models import f64_hex, hex_array


def _f64(hex_text: str) -> float:
    return struct.unpack(">d", bytes.fromhex(hex_text))[0]


def _clock_steps(d: dict, ticks: int) -> list[int]:
    """Each clock's ticks in `ticks` ticks of the first (default) clock; every clock must
    advance a whole number of its own ticks in that time."""
    dt0 = _f64(d["clocks"][0]["dt"])
    out = []
    for clock in d["clocks"]:
        exact = ticks * dt0 / _f64(clock["dt"])
        steps = int(round(exact))
        if abs(exact - steps) > 1e-9 * max(1.0, exact):
            raise ValueError("a segment boundary must fall on a tick of every clock")
        out.append(steps)
    return out


def _pathway_clock(d: dict, sdef: dict, pathway: dict) -> int:
    """The clock a pathway runs on: that of the population whose events trigger it."""
    endpoint = "source" if pathway["kind"] == "pre" else "target"
    return int(d["populations"][sdef[f"{endpoint}_population"]]["clock"])


def first_segment(document: dict, ticks: int) -> dict:
    """The sealed document running only the first `ticks` ticks (of the default clock) of
    `document`."""
    doc = copy.deepcopy(protocol.load(document, verify_envelope=False))
    doc.pop("protocol", None)
    d, run = doc["definition"], doc["run"]
    if not 0 < ticks <= int(run["clocks"][0]["steps"]):
        raise ValueError("a first segment runs between 1 tick and the whole run")
    steps = _clock_steps(d, ticks)
    run["duration"] = f64_hex(ticks * _f64(d["clocks"][0]["dt"]))
    for c, clock in enumerate(run["clocks"]):
        clock["steps"] = steps[c]
    for pdef in d["populations"]:
        mine = steps[int(pdef["clock"])]
        pdef["steps"] = mine
        pdef["monitor"]["window_steps"] = min(int(pdef["monitor"]["window_steps"]), mine)
    for sdef, sin in zip(d["synapses"], doc["instance"]["synapses"]):
        for pathway in sin["pathways"]:
            c = _pathway_clock(d, sdef, pathway)
            end = int(run["clocks"][c]["start_tick"]) + steps[c]
            if any(int(e["delivery_tick"]) >= end for e in pathway.get("pending", [])):
                raise ValueError("pending events arrive after the end of the segment")
    return protocol.seal(doc)


def continuation(document: dict, result: dict, ticks: int) -> dict:
    """The sealed AtlasIR document running `ticks` more ticks (of the default clock) after the run
    of `document` whose result (HipExecutor.run() dictionary) is `result`.  With several clocks
    each clock continues from its own end tick, and each pathway's pending events count the ticks
    of the clock it runs on."""
    doc = copy.deepcopy(protocol.load(document, verify_envelope=False))
    doc.pop("protocol", None)
    d, inst, run = doc["definition"], doc["instance"], doc["run"]
    dt = _f64(d["clocks"][0]["dt"])
    steps = _clock_steps(d, int(ticks))
    old_steps = [int(clock["steps"]) for clock in run["clocks"]]
    ends = [int(clock["start_tick"]) + int(clock["steps"]) for clock in run["clocks"]]
    run["start"] = f64_hex(_f64(run["start"]) + _f64(run["duration"]))
    run["duration"] = f64_hex(ticks * dt)
    run["clocks"] = [{"start_tick": ends[c], "steps": steps[c]} for c in range(len(run["clocks"]))]
    for pdef, pin, pres in zip(d["populations"], inst["populations"], result["populations"]):
        c = int(pdef["clock"])
        end_tick, new_end = ends[c], ends[c] + steps[c]
        pdef["steps"] = steps[c]
        pdef["monitor"]["window_steps"] = min(int(pdef["monitor"]["window_steps"]), steps[c])
        for symbol in pdef["states"]:
            pin["initial_state"][symbol["name"]] = hex_array(pres["states"][symbol["name"]], symbol["dtype"])
        if pin.get("refractory") is not None:
            refractory = pres["refractory"]
            pin["refractory"]["initial_lastspike"] = hex_array(refractory["lastspike"], "f64")
            pin["refractory"]["initial_not_refractory"] = [bool(v) for v in refractory["not_refractory"]]
        generator = pin.get("spike_generator")
        if generator is not None:
            keep = [k for k, t in enumerate(generator["spike_ticks"]) if end_tick <= int(t) < new_end]
            pin["spike_generator"] = {"spike_ticks": [int(generator["spike_ticks"][k]) for k in keep],
                                      "spike_indices": [int(generator["spike_indices"][k]) for k in keep]}
    for sdef, sin, sres in zip(d["synapses"], inst["synapses"], result["synapses"]):
        for symbol in sdef["states"]:
            sin["initial_state"][symbol["name"]] = hex_array(sres["states"][symbol["name"]], symbol["dtype"])
        explicit = sin.get("topology", {"kind": "explicit"})["kind"] == "explicit"
        for pathway in sin["pathways"]:
            endpoint = "source" if pathway["kind"] == "pre" else "target"
            population = sdef[f"{endpoint}_population"]
            c = _pathway_clock(d, sdef, pathway)
            end_tick, new_end, old_clock_steps = ends[c], ends[c] + steps[c], old_steps[c]
            start, count = sdef[f"{endpoint}_start"], sdef[f"{endpoint}_count"]
            window = d["populations"][population]["monitor"]["window_steps"]
            delays = [int(v) for v in pathway["delay_ticks"]]
            retained = [dict(e) for e in pathway.get("pending", []) if int(e["delivery_tick"]) >= end_tick]
            if delays and max(delays) > 0 and old_clock_steps > window and window < max(delays):
                raise ValueError("the recording window does not cover the pending delays")
            stream = result["populations"][population]["event_streams"][pathway["event"]]
            ticks_, indices = stream["ticks"], stream["indices"]
            ticks_ = np.asarray(ticks_, np.int64)
            local = np.asarray(indices, np.int64) - start
            inside = (local >= 0) & (local < count)
            new = []
            if delays and all(v == delays[0] for v in delays):
                chosen = inside & (ticks_ + delays[0] >= end_tick)
                new = [{"delivery_tick": int(t) + delays[0], "item": int(i)}
                       for t, i in zip(ticks_[chosen], local[chosen])]
            elif delays:
                if not explicit:
                    raise ValueError("per-edge delays continue only with explicit topologies")
                endpoints = np.asarray(sin[endpoint], np.int64)
                delay_of = np.asarray(delays, np.int64)
                chosen = inside & (ticks_ + delay_of.max() >= end_tick)
                for t, i in zip(ticks_[chosen], local[chosen]):
                    for edge in np.flatnonzero(endpoints == i):
                        delivery = int(t) + int(delay_of[edge])
                        if delivery >= end_tick:
                            new.append({"delivery_tick": delivery, "item": int(edge)})
            pending = retained + new
            pending.sort(key=lambda event: event["delivery_tick"])
            pathway["pending"] = [e for e in pending if e["delivery_tick"] < new_end]
    return protocol.seal(doc)
