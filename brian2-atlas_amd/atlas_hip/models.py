"""AtlasIR v1 documents for the benchmark networks, written without Brian2.

Brian2 is not available on the GPU host, so the configurations are built here as
AtlasIR documents with the structure the Atlas exporter emits:

* statement trees follow the exporter's typing rules (``spec.py:900-975``): loads
  of float32 states are widened with ``f32_to_f64``, every assignment to a
  float32 target is narrowed once with ``f64_to_f32``;
* dimensioned namespace constants are scalar f64 parameters (as ``ms`` in the
  reference fixture ``tests/fixtures/reference-v1/model.json``);
* schedule nodes are sorted by ``(slot, order, name, id)`` and carry their
  resource effects and the transitive reduction of the RAW/WAR/WAW conflicts
  with earlier nodes (AtlasIR.md section 5);
* Bernoulli ``connect(condition, p)`` replays the exporter's NumPy legacy
  MT19937 draw order: one ``random(N_target)`` row per source, drawn even for
  rows the condition rejects (``device.py:1032-1048``); ``rand()`` string
  initialisers draw ``np.random.rand(N)``;
* procedural ``fixed_indegree`` projections carry the seed derivation of
  ``connect_fixed_indegree`` (``device.py:299-302``) and initializer streams
  ``2 + 2k`` (``export.py:2386-2403``); uniform delays collapse to one entry
  (``export.py:2417-2419``).

Bit-exactness is defined relative to a document: the oracle and the HIP engine
execute the same statement trees.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

import numpy as np

from . import protocol

SLOTS = ["start", "groups", "thresholds", "synapses", "resets", "end"]
EXPANDED = [f"{prefix}{slot}" for slot in SLOTS for prefix in ("before_", "", "after_")]
DIMLESS = [0.0] * 7
SECOND = [0.0, 0.0, 1.0, 0.0, 0.0, 0.0, 0.0]
VOLT = [2.0, 1.0, -3.0, -1.0, 0.0, 0.0, 0.0]
SIEMENS = [-2.0, -1.0, 3.0, 2.0, 0.0, 0.0, 0.0]
FARAD = [-2.0, -1.0, 4.0, 2.0, 0.0, 0.0, 0.0]
AMP = [0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0]


# -------------------------------------------------------------------- encodings
def f64_hex(value: float) -> str:
    return struct.pack(">d", float(value)).hex()


def f32_hex(value: float) -> str:
    return struct.pack(">f", float(value)).hex()


def hex_array(values, dtype: str) -> list[str]:
    """Vectorised AtlasIR encoding of a numeric array (AtlasIR.md section 3)."""
    arr = np.asarray(values)
    if dtype == "f64":
        raw, width = arr.astype(">f8").tobytes().hex(), 16
    elif dtype == "f32":
        raw, width = arr.astype(">f4").tobytes().hex(), 8
    elif dtype == "bool":
        return ["01" if v else "00" for v in arr.astype(bool)]
    elif dtype in ("i32", "u32"):
        raw, width = arr.astype(">u4" if dtype == "u32" else ">i4").tobytes().hex(), 8
    else:
        raw, width = arr.astype(">u8" if dtype == "u64" else ">i8").tobytes().hex(), 16
    return [raw[k:k + width] for k in range(0, len(raw), width)]


# ------------------------------------------------------------------ expressions
def lit(value: float) -> dict:
    return {"op": "literal", "bits": f64_hex(value)}


def integer(value: int, dtype: str = "i64") -> dict:
    return {"op": "integer", "dtype": dtype, "value": str(int(value))}


def ld(name: str) -> dict:
    return {"op": "load", "name": name}


def wide(expr: dict) -> dict:
    return {"op": "f32_to_f64", "arg": expr}


def narrow(expr: dict) -> dict:
    return {"op": "f64_to_f32", "arg": expr}


def op(name: str, left: dict, right: dict) -> dict:
    return {"op": name, "left": left, "right": right}


def un(name: str, arg: dict) -> dict:
    return {"op": name, "arg": arg}


def add(a, b): return op("add", a, b)
def sub(a, b): return op("sub", a, b)
def mul(a, b): return op("mul", a, b)
def div(a, b): return op("div", a, b)
def neg(a): return un("neg", a)


def initializer_uniform(minimum: float, maximum: float) -> dict:
    """A procedural per-edge ``Uniform(minimum, maximum)`` initializer (model.rs:465-530);
    the stream is assigned by ``NetworkBuilder.projection``."""
    return {"kind": "uniform", "minimum": f64_hex(minimum), "maximum": f64_hex(maximum)}


def initializer_clipped_normal(mean: float, std: float, minimum: float | None = None,
                               maximum: float | None = None) -> dict:
    """A procedural per-edge ``ClippedNormal(mean, std, minimum, maximum)`` initializer."""
    return {"kind": "clipped_normal", "mean": f64_hex(mean), "std": f64_hex(std),
            "minimum": None if minimum is None else f64_hex(minimum),
            "maximum": None if maximum is None else f64_hex(maximum)}


def stmt(target: str, dtype: str, value: dict, dims=DIMLESS, condition: str | None = None) -> dict:
    return {"target": target, "dtype": dtype, "dimensions": list(dims), "value": value,
            "condition": condition}


def _loads(expr, out: set) -> None:
    if isinstance(expr, dict):
        if expr.get("op") == "load":
            out.add(expr["name"])
        for value in expr.values():
            _loads(value, out)
    elif isinstance(expr, list):
        for value in expr:
            _loads(value, out)


def code_effects(scalar: list, vector: list, writable: set) -> dict:
    reads: set = set()
    defined: set = set()
    writes: set = set()
    for statement in scalar + vector:
        found: set = set()
        _loads(statement["value"], found)
        if statement.get("condition"):
            found.add(statement["condition"])
        reads |= {name for name in found if name not in defined}
        defined.add(statement["target"])
        if statement["target"] in writable:
            writes.add(statement["target"])
    return {"reads": sorted(reads), "writes": sorted(writes)}


# ---------------------------------------------------------------------- builder
@dataclass
class _Population:
    definition: dict
    instance: dict


@dataclass
class NetworkBuilder:
    """Accumulates populations, projections and monitors, then emits AtlasIR."""

    dt: float = 1e-4
    steps: int = 10000
    seed: int = 1729
    populations: list = field(default_factory=list)
    synapses: list = field(default_factory=list)
    procedural_count: int = 0
    packed: bool = False       # keep arrays as numpy (in-memory large-array documents, not serialisable)
    extra_clocks: list = field(default_factory=list)   # (dt, steps) of clocks 1, 2, ...

    def add_clock(self, dt: float) -> int:
        """A further clock of step ``dt`` for the run's duration (steps * the default dt), which
        must be a whole number of its ticks; returns its index for ``population(clock=...)``."""
        ticks = self.steps * self.dt / dt
        steps = int(round(ticks))
        if abs(ticks - steps) > 1e-9 * max(1.0, ticks):
            raise ValueError("the run's duration is not a whole number of ticks of the clock")
        self.extra_clocks.append((float(dt), steps))
        return len(self.extra_clocks)

    def clock_of(self, clock: int) -> tuple[float, int]:
        return (self.dt, self.steps) if clock == 0 else self.extra_clocks[clock - 1]

    def _enc(self, values, dtype: str):
        if self.packed:
            storage = {"f64": np.float64, "f32": np.float32, "bool": np.uint8, "i32": np.int32, "u32": np.uint32,
                       "i64": np.int64, "u64": np.uint64}[dtype]
            return np.ascontiguousarray(np.asarray(values).reshape(-1).astype(storage, copy=False))
        return hex_array(values, dtype)

    # populations --------------------------------------------------------------
    def population(self, name: str, count: int, *, states: dict, parameters: dict | None = None,
                   update: tuple[list, list] | None = None, threshold: dict | None = None,
                   reset: list | None = None, refractory: float | None = None,
                   frozen: tuple = ("v",), spike_monitor: bool = True,
                   state_monitor: tuple[list, list] | None = None, event_monitor: list | None = None,
                   clock: int = 0, custom_events: dict | None = None, event_monitors: list | None = None) -> int:
        """Add a NeuronGroup.

        ``states`` maps name -> (dtype, dims, initial array); ``parameters`` maps
        name -> (dtype, dims, value) for scalars or (dtype, dims, array) per neuron.
        ``custom_events`` maps an event's name -> (condition, run_on_event statements or None), as
        NeuronGroup(events=...) and run_on_event declare them; ``event_monitors`` lists further
        EventMonitors as (event, variables, when) with ``when`` "thresholds" or "end".
        """
        index = len(self.populations)
        offset = sum(p.definition["count"] for p in self.populations)
        parameters = parameters or {}
        state_syms = [{"name": k, "dtype": v[0], "dimensions": list(v[1]), "index_domain": "neuron"}
                      for k, v in states.items()]
        param_syms = []
        param_values = {}
        for k, (dtype, dims, value) in parameters.items():
            scalar = np.ndim(value) == 0
            param_syms.append({"name": k, "dtype": dtype, "dimensions": list(dims),
                               "index_domain": "scalar" if scalar else "neuron"})
            param_values[k] = self._enc([value] if scalar else value, dtype)
        writable = set(states) | ({"not_refractory"} if refractory is not None else set())
        codes = []
        events = []
        if update is not None:
            scalar, vector = update
            codes.append({"name": f"{name}_stateupdater", "kind": "state_update", "when": "groups",
                          "order": 0, "clock": 0, "iteration_domain": "all_neurons",
                          "scalar": scalar, "vector": vector,
                          "effects": code_effects(scalar, vector, writable)})
        if threshold is not None:
            events.append("spike")
            vector = [stmt("_cond", "bool", threshold)]
            codes.append({"name": f"{name}_spike_thresholder", "kind": "threshold",
                          "when": "thresholds", "order": 0, "clock": 0,
                          "iteration_domain": "all_neurons", "scalar": [], "vector": vector,
                          "effects": code_effects([], vector, writable), "event_name": "spike"})
        if reset is not None:
            codes.append({"name": f"{name}_spike_resetter", "kind": "reset", "when": "resets",
                          "order": 0, "clock": 0, "iteration_domain": "spiking_neurons",
                          "scalar": [], "vector": reset,
                          "effects": code_effects([], reset, writable), "event_name": "spike"})
        for event, (condition, on_event) in (custom_events or {}).items():
            vector = [stmt("_cond", "bool", condition)]
            codes.append({"name": f"{name}_{event}_thresholder", "kind": "threshold",
                          "when": "thresholds", "order": 0, "clock": 0,
                          "iteration_domain": "all_neurons", "scalar": [], "vector": vector,
                          "effects": code_effects([], vector, writable), "event_name": event})
            if on_event is not None:
                codes.append({"name": f"{name}_{event}_resetter", "kind": "reset", "when": "resets",
                              "order": 0, "clock": 0, "iteration_domain": "spiking_neurons",
                              "scalar": [], "vector": on_event,
                              "effects": code_effects([], on_event, writable), "event_name": event})
        record_vars, record_idx = state_monitor if state_monitor else ([], [])
        definition = {
            "name": name, "offset": offset, "count": count, "states": state_syms,
            "parameters": param_syms, "linked_variables": [],
            "refractory": ({"frozen_states": list(frozen), "mode": "fixed"}
                           if refractory is not None else None),
            "events": events + list(custom_events or {}), "code_objects": codes,
            "state_monitors": ([{"name": f"{name}_statemonitor", "variables": list(record_vars),
                                 "record": [int(i) for i in record_idx], "clock": 0}]
                               if state_monitor else []),
            "event_monitors": ([{"name": f"{name}_eventmonitor", "event": "spike", "variables": list(event_monitor),
                                 "clock": 0, "when": "thresholds", "order": 1}] if event_monitor is not None else []) +
                              [{"name": f"{name}_{event}_{when}_eventmonitor{k}", "event": event,
                                "variables": list(variables), "clock": 0, "when": when, "order": 1}
                               for k, (event, variables, when) in enumerate(event_monitors or [])],
            "spike_monitor": f"{name}_spikemonitor" if spike_monitor and threshold is not None else None,
            "monitor": {"variables": list(record_vars), "record": [int(i) for i in record_idx],
                        "window_steps": self.steps},
            "clock": 0, "dt": f64_hex(self.dt), "steps": self.steps,
        }
        # the population, its code objects and monitors on one clock
        dt, steps = self.clock_of(clock)
        definition.update(clock=clock, dt=f64_hex(dt), steps=steps)
        definition["monitor"]["window_steps"] = steps
        for item in definition["code_objects"] + definition["state_monitors"] + definition["event_monitors"]:
            item["clock"] = clock
        refr_instance = None
        if refractory is not None:
            period_ticks = int((refractory + 1e-3 * dt) / dt)
            refr_instance = {"period": f64_hex(refractory), "period_ticks": period_ticks,
                             "initial_lastspike": self._enc(np.full(count, -1e4), "f64"),
                             "initial_not_refractory": [True] * count}
        instance = {"initial_state": {k: self._enc(v[2], v[0]) for k, v in states.items()},
                    "parameters": param_values, "refractory": refr_instance, "spike_generator": None}
        self.populations.append(_Population(definition, instance))
        return index

    def spike_generator(self, name: str, count: int, ticks, indices, *, spike_monitor: bool = True,
                        clock: int = 0) -> int:
        """Add a SpikeGeneratorGroup as the reference exporter lowers it (export.py:1324-1410): no
        states or code objects, the (tick, neuron) schedule, in ticks of its clock, sorted in the
        instance."""
        pairs = sorted(zip((int(t) for t in ticks), (int(i) for i in indices)))
        index = self.population(name, count, states={}, spike_monitor=False, clock=clock)
        pop = self.populations[index]
        pop.definition["events"] = ["spike"]
        pop.definition["spike_monitor"] = f"{name}_spikemonitor" if spike_monitor else None
        pop.instance["spike_generator"] = {"spike_ticks": [t for t, _ in pairs], "spike_indices": [i for _, i in pairs]}
        return index

    def poisson_input(self, population: int, target: str, n: int, rate: float, weight: float,
                      *, name: str | None = None) -> int:
        """Add a PoissonInput as the reference exporter lowers it (export.py:571-608, 845-858):
        a ``poisson_input`` code object in the synapses slot at order 0 whose statement is
        ``target += binomial(n, p) * weight`` (binomial with the normal approximation, on its
        own random stream), p = rate * dt in the scalar parameter
        ``b2_poisson_probability_<k>``."""
        pop = self.populations[population]
        d, inst = pop.definition, pop.instance
        k = sum(1 for c in d["code_objects"] if c["kind"] == "poisson_input")
        pname = f"b2_poisson_probability_{k}"
        d["parameters"].append({"name": pname, "dtype": "f64", "dimensions": list(DIMLESS), "index_domain": "scalar"})
        inst["parameters"][pname] = self._enc([float(rate) * self.clock_of(d["clock"])[0]], "f64")
        symbol = next(s_ for s_ in d["states"] if s_["name"] == target)
        draw = {"op": "binomial", "stream": 1000 + k, "n": int(n), "p": ld(pname), "approximate": True}
        f32 = symbol["dtype"] == "f32"
        value = add(wide(ld(target)) if f32 else ld(target), mul(draw, lit(weight)))
        vector = [stmt(target, symbol["dtype"], narrow(value) if f32 else value, tuple(symbol["dimensions"]))]
        writable = {s_["name"] for s_ in d["states"]}
        d["code_objects"].append({"name": name or f"{d['name']}_poissoninput_{k}", "kind": "poisson_input",
                                  "when": "synapses", "order": 0, "clock": d["clock"], "iteration_domain": "all_neurons",
                                  "scalar": [], "vector": vector, "effects": code_effects([], vector, writable)})
        return k

    def run_regularly(self, population: int, vector: list, *, scalar: list = (), when: str = "start",
                      order: int = 0, name: str | None = None) -> int:
        """Add a ``run_regularly`` code object (a stateless CodeRunner of the population, on its
        clock, export.py:612): ``vector`` statements over every neuron at the node's schedule
        slot ``when`` (Brian2's default "start") and ``order``."""
        pop = self.populations[population]
        d = pop.definition
        k = sum(1 for c in d["code_objects"] if c["kind"] == "run_regularly")
        writable = {s_["name"] for s_ in d["states"]}
        d["code_objects"].append({"name": name or f"{d['name']}_run_regularly_{k}", "kind": "run_regularly",
                                  "when": when, "order": int(order), "clock": d["clock"],
                                  "iteration_domain": "all_neurons", "scalar": list(scalar), "vector": list(vector),
                                  "effects": code_effects(list(scalar), list(vector), writable)})
        return k

    # synapses -----------------------------------------------------------------
    def projection(self, name: str, source: int, target: int, *, on_pre: list,
                   source_range: tuple[int, int] | None = None,
                   target_range: tuple[int, int] | None = None,
                   pre_aliases: dict | None = None, post_aliases: dict | None = None,
                   states: dict | None = None, parameters: dict | None = None,
                   on_post: list | None = None, explicit: tuple | None = None,
                   fixed_indegree: int | None = None, fixed_total: int | None = None,
                   topology_seed: int | None = None, initializers: dict | None = None,
                   delay_ticks=0, delay_initializer: dict | None = None, post_delay_ticks: int = 0,
                   clock_driven: list | None = None, summed: list | None = None,
                   pre_events: dict | None = None, post_event: str = "spike") -> int:
        """Add a Synapses object with one ``pre`` (and optionally one ``post``) pathway.

        ``on_pre`` may instead map pathway names to their statements (several on_pre pathways,
        ordered by name); ``pre_events`` then names the source event that triggers each (default
        "spike"), and ``delay_ticks`` may map the names to their delays.  ``post_event`` names the
        target event that triggers on_post.

        ``explicit`` = (source array, target array) in creation order, local to the
        source/target ranges; ``fixed_indegree`` = K or ``fixed_total`` = E uses a
        procedural topology (connect_fixed_indegree / connect_fixed_total), seeded with
        ``topology_seed`` or a seed derived from the network seed.  ``initializers``
        maps per-edge parameters to procedural initializers (``initializer_uniform`` /
        ``initializer_clipped_normal``), numbered on streams 2, 4, ... in name order,
        and ``delay_initializer`` draws the on_pre delays (in seconds) on the next
        stream, as the reference frontend numbers them.
        ``delay_ticks`` is a scalar tick count or a per-edge array (on_pre);
        ``post_delay_ticks`` the delay of the on_post pathway (uniform, or one per edge).
        ``clock_driven`` are the statements of the synapse state update (the states they assign
        are the clock-driven states); ``summed`` lists summed variables as (population state,
        expression of ``_synaptic_var``, endpoint "post" or "pre"), in the groups slot before
        the neuron updates.
        """
        index = len(self.synapses)
        spop = self.populations[source].definition
        tpop = self.populations[target].definition
        s0, s1 = source_range or (0, spop["count"])
        t0, t1 = target_range or (0, tpop["count"])
        states = states or {}
        parameters = parameters or {}
        pre_aliases = pre_aliases or {}
        post_aliases = post_aliases or {}
        state_syms = [{"name": k, "dtype": v[0], "dimensions": list(v[1]), "index_domain": "synapse"}
                      for k, v in states.items()]
        param_syms, param_values = [], {}
        for k, (dtype, dims, value) in parameters.items():
            # a value of None declares a per-edge parameter drawn by a procedural initializer
            scalar = value is not None and np.ndim(value) == 0
            param_syms.append({"name": k, "dtype": dtype, "dimensions": list(dims),
                               "index_domain": "scalar" if scalar else "synapse"})
            if value is not None:
                param_values[k] = self._enc([value] if scalar else value, dtype)
        writable = set(states) | set(post_aliases) | set(pre_aliases)
        # code objects in the reference's order: summed variables, the state update, pathways
        # (model.rs:4394-4455)
        codes = []
        for state, expression, endpoint in summed or []:
            full = (s0, s1) == (0, spop["count"]) if endpoint == "pre" else (t0, t1) == (0, tpop["count"])
            vector = [stmt("_synaptic_var", "f64", expression)]
            codes.append({"name": f"{name}_summed_variable_{state}_{endpoint}", "kind": "summed_variable",
                          "when": "groups", "order": -1 if full else 0, "clock": 0,
                          "iteration_domain": "all_synapses", "scalar": [], "vector": vector,
                          "effects": code_effects([], vector, set()), "pathway_name": None, "event_name": None,
                          "summed_target": endpoint, "summed_state": state})
        clock_driven_states = []
        if clock_driven:
            clock_driven_states = sorted({st["target"] for st in clock_driven} & set(states))
            codes.append({"name": f"{name}_stateupdater", "kind": "synapse_state_update", "when": "groups",
                          "order": 0, "clock": 0, "iteration_domain": "all_synapses", "scalar": [],
                          "vector": clock_driven, "effects": code_effects([], clock_driven, set(clock_driven_states)),
                          "pathway_name": None, "event_name": None})
        pre_paths = sorted(on_pre.items()) if isinstance(on_pre, dict) else [("pre", on_pre)]
        for key, statements in pre_paths:
            codes.append({"name": f"{name}_{key}", "kind": "synapses", "when": "synapses", "order": -1,
                          "clock": 0, "iteration_domain": "active_synapses", "scalar": [], "vector": statements,
                          "effects": code_effects([], statements, writable), "pathway_name": f"{name}_{key}",
                          "event_name": (pre_events or {}).get(key, "spike")})
        if on_post is not None:
            codes.append({"name": f"{name}_post", "kind": "synapses_post", "when": "synapses",
                          "order": 1, "clock": 0, "iteration_domain": "active_synapses",
                          "scalar": [], "vector": on_post,
                          "effects": code_effects([], on_post, set(states) | set(post_aliases)),
                          "pathway_name": f"{name}_post", "event_name": post_event})
        # on_pre code runs on the source's clock, on_post code and summed variables into the
        # targets on the target's
        sclock, tclock = spop["clock"], tpop["clock"]
        for code in codes:
            post_side = code["kind"] == "synapses_post" or (code["kind"] == "summed_variable"
                                                              and code["summed_target"] == "post")
            code["clock"] = tclock if post_side else sclock
        definition = {"name": name, "states": state_syms, "clock_driven_states": clock_driven_states,
                      "parameters": param_syms, "pre_state_aliases": dict(pre_aliases),
                      "post_state_aliases": dict(post_aliases), "source_population": source,
                      "target_population": target, "source_start": s0, "target_start": t0,
                      "source_count": s1 - s0, "target_count": t1 - t0, "code_objects": codes}
        if explicit is not None:
            src, tgt = explicit
            edge_count = len(src)
            topology = {"kind": "explicit"}
            if self.packed:
                sources = np.ascontiguousarray(np.asarray(src, np.int64))
                targets = np.ascontiguousarray(np.asarray(tgt, np.int64))
            else:
                sources = [int(v) for v in np.asarray(src)]
                targets = [int(v) for v in np.asarray(tgt)]
        else:
            self.procedural_count += 1
            seed = (self.seed ^ (self.procedural_count * 0x9E3779B97F4A7C15)) & (2**64 - 1)
            if topology_seed is not None:
                seed = int(topology_seed)
            inits = {}
            for position, key in enumerate(sorted(initializers or {})):
                inits[key] = dict(initializers[key], stream=2 + 2 * position)
            if fixed_total is not None:
                edge_count = int(fixed_total)
                topology = {"kind": "fixed_total", "edge_count": edge_count, "seed": seed, "initializers": inits}
            else:
                edge_count = fixed_indegree * (t1 - t0)
                topology = {"kind": "fixed_indegree", "edge_count": edge_count,
                            "indegree": int(fixed_indegree), "seed": seed, "initializers": inits}
            sources, targets = [], []
        pathways = []
        pathway_kinds = [("pre", f"{name}_{key}", key) for key, _ in pre_paths] + \
            ([("post", f"{name}_post", "post")] if on_post else [])
        n_inits = len(topology.get("initializers", {}))
        for position, (kind, pname, key) in enumerate(pathway_kinds):
            pre_delays = delay_ticks.get(key, 0) if isinstance(delay_ticks, dict) else delay_ticks
            delays = np.atleast_1d(np.asarray(pre_delays if kind == "pre" else post_delay_ticks, dtype=np.int64))
            if delays.size == edge_count and edge_count and np.all(delays == delays[0]):
                delays = delays[:1]
            descriptor = None
            if delay_initializer is not None and kind == "pre":
                descriptor = dict(delay_initializer, stream=2 + 2 * n_inits + 2 * position)
                delays = np.zeros(0, np.int64)
            pathway_dt = self.clock_of(sclock if kind == "pre" else tclock)[0]
            event = (pre_events or {}).get(key, "spike") if kind == "pre" else post_event
            pathways.append({"name": pname, "kind": kind, "event": event,
                             "delay": self._enc(delays * pathway_dt, "f64"),
                             "delay_ticks": delays if self.packed else [int(v) for v in delays],
                             "delay_initializer": descriptor, "pending": []})
        instance = {"source": sources, "target": targets, "topology": topology,
                    "initial_state": {k: self._enc(v[2], v[0]) for k, v in states.items()},
                    "parameters": param_values, "pathways": pathways}
        self.synapses.append((definition, instance))
        return index

    # document -------------------------------------------------------------------
    def _resource(self, owner: str, index: int, name: str, pop_states: set, pop_params: set) -> str | None:
        if name in ("dt", "t", "N", "i", "j", "N_pre", "N_post", "lastspike"):
            return None
        if name == "not_refractory":
            return f"{owner}/{index}/refractory/not_refractory"
        if name in pop_states:
            return f"{owner}/{index}/state/{name}"
        if name in pop_params:
            return f"{owner}/{index}/parameter/{name}"
        return None

    def _schedule(self) -> dict:
        nodes = []
        for p, pop in enumerate(self.populations):
            d = pop.definition
            states = {s["name"] for s in d["states"]}
            params = {s["name"] for s in d["parameters"]}
            res = lambda n: self._resource("population", p, n, states, params)  # noqa: E731
            for k, monitor in enumerate(d["state_monitors"]):
                nodes.append({"id": f"population/{p}/state_monitor/{k}", "operation": "state_monitor",
                              "owner_kind": "population", "owner_index": p, "item_index": k,
                              "clock": monitor["clock"], "when": "start", "order": 0, "name": monitor["name"],
                              "reads": {res(v) for v in monitor["variables"]} - {None}, "writes": set()})
            for k, code in enumerate(d["code_objects"]):
                reads = {res(n) for n in code["effects"]["reads"]} - {None}
                writes = {res(n) for n in code["effects"]["writes"]} - {None}
                if code["kind"] == "threshold":
                    writes.add(f"population/{p}/event/{code['event_name']}")
                if code["kind"] == "reset":
                    reads.add(f"population/{p}/event/{code['event_name']}")
                nodes.append({"id": f"population/{p}/code/{k}", "operation": "code_object",
                              "owner_kind": "population", "owner_index": p, "item_index": k,
                              "clock": code["clock"], "when": code["when"], "order": code["order"],
                              "name": code["name"], "reads": reads, "writes": writes})
            for k, monitor in enumerate(d["event_monitors"]):
                nodes.append({"id": f"population/{p}/event_monitor/{k}", "operation": "event_monitor",
                              "owner_kind": "population", "owner_index": p, "item_index": k,
                              "clock": monitor["clock"], "when": monitor["when"], "order": monitor["order"],
                              "name": monitor["name"],
                              "reads": {f"population/{p}/event/{monitor['event']}"} |
                                       ({res(v) for v in monitor["variables"]} - {None}), "writes": set()})
            if pop.instance.get("spike_generator") is not None:
                nodes.append({"id": f"population/{p}/event_source/0", "operation": "event_source",
                              "owner_kind": "population", "owner_index": p, "item_index": 0,
                              "clock": d["clock"], "when": "thresholds", "order": 0, "name": d["name"],
                              "reads": set(), "writes": {f"population/{p}/event/spike"}})
            if d["spike_monitor"]:
                nodes.append({"id": f"population/{p}/spike_monitor/0", "operation": "spike_monitor",
                              "owner_kind": "population", "owner_index": p, "item_index": 0,
                              "clock": d["clock"], "when": "thresholds", "order": 1, "name": d["spike_monitor"],
                              "reads": {f"population/{p}/event/spike"}, "writes": set()})
        for s, (d, _inst) in enumerate(self.synapses):
            sp, tp = d["source_population"], d["target_population"]
            tdef = self.populations[tp].definition
            syn_states = {x["name"] for x in d["states"]}
            syn_params = {x["name"] for x in d["parameters"]}
            for k, code in enumerate(d["code_objects"]):
                reads, writes = set(), set()
                if code["kind"] in ("synapses", "synapses_post"):
                    event_pop = sp if code["kind"] == "synapses" else tp
                    reads.add(f"population/{event_pop}/event/{code['event_name']}")
                if code["kind"] == "summed_variable":
                    endpoint = sp if code["summed_target"] == "pre" else tp
                    writes.add(f"population/{endpoint}/state/{code['summed_state']}")
                for names, out in ((code["effects"]["reads"], reads), (code["effects"]["writes"], writes)):
                    for n in names:
                        if n in syn_states:
                            out.add(f"synapse/{s}/state/{n}")
                        elif n in syn_params:
                            out.add(f"synapse/{s}/parameter/{n}")
                        elif n in d["post_state_aliases"]:
                            out.add(f"population/{tp}/state/{d['post_state_aliases'][n]}")
                        elif n in d["pre_state_aliases"]:
                            out.add(f"population/{sp}/state/{d['pre_state_aliases'][n]}")
                        elif n == "not_refractory_post" and tdef["refractory"] is not None:
                            out.add(f"population/{tp}/refractory/not_refractory")
                nodes.append({"id": f"synapse/{s}/code/{k}", "operation": "code_object",
                              "owner_kind": "synapse", "owner_index": s, "item_index": k,
                              "clock": code["clock"], "when": code["when"], "order": code["order"],
                              "name": code["name"], "reads": reads, "writes": writes})
        slot_rank = {name: position for position, name in enumerate(EXPANDED)}
        nodes.sort(key=lambda n: (slot_rank[n["when"]], n["order"], n["name"], n["id"]))
        ancestors: dict[str, set] = {}
        for k, node in enumerate(nodes):
            conflicts = []
            for earlier in nodes[:k]:
                if (earlier["writes"] & node["reads"]) or (earlier["reads"] & node["writes"]) or \
                        (earlier["writes"] & node["writes"]):
                    conflicts.append(earlier["id"])
            reachable = set()
            for dep in conflicts:
                reachable |= ancestors[dep]
            node["dependencies"] = sorted(dep for dep in conflicts if dep not in reachable)
            ancestors[node["id"]] = set(conflicts) | reachable
        out = []
        for node in nodes:
            node["effects"] = {"reads": sorted(node.pop("reads")), "writes": sorted(node.pop("writes"))}
            out.append(node)
        return {"base_slots": SLOTS, "slots": EXPANDED, "nodes": out}

    def document(self) -> dict:
        definition = {
            "clocks": [{"name": "defaultclock", "dt": f64_hex(self.dt)}] +
                      [{"name": f"clock_{k + 1}", "dt": f64_hex(dt)} for k, (dt, _) in enumerate(self.extra_clocks)],
            "populations": [p.definition for p in self.populations],
            "synapses": [s[0] for s in self.synapses],
            "functions": [],
            "schedule": self._schedule(),
            "numeric_profile": "reference-f64",
            "rng_algorithm": "splitmix64-counter-v1",
        }
        instance = {"neuron_count": sum(p.definition["count"] for p in self.populations),
                    "populations": [p.instance for p in self.populations],
                    "synapses": [s[1] for s in self.synapses], "rng_seed": int(self.seed)}
        run = {"start": f64_hex(0.0), "duration": f64_hex(self.steps * self.dt),
               "clocks": [{"start_tick": 0, "steps": self.steps}] +
                         [{"start_tick": 0, "steps": steps} for _, steps in self.extra_clocks]}
        document = {"schema": protocol.CURRENT_SCHEMA, "definition": definition, "instance": instance, "run": run}
        # a packed document holds numpy arrays: it has no canonical JSON and no envelope
        return document if self.packed else protocol.seal(document)


# ------------------------------------------------------------------- CUBA family
def cuba_update(dtype: str = "f32") -> tuple[list, list]:
    """Exact (matrix-exponential) update of the CUBA equations (examples/CUBA.py:24-28).

    dv/dt = (ge + gi - (v - El))/taum (unless refractory), dge/dt = -ge/taue,
    dgi/dt = -gi/taui.  Loop invariants are hoisted into scalar ``_lio_*``
    statements as the Brian code generator does.
    """
    w = wide if dtype == "f32" else (lambda e: e)
    n = narrow if dtype == "f32" else (lambda e: e)
    em = un("exp", div(neg(ld("dt")), ld("taum")))
    ee = un("exp", div(neg(ld("dt")), ld("taue")))
    ei = un("exp", div(neg(ld("dt")), ld("taui")))
    scalar = [
        stmt("_lio_1", "f64", em),
        stmt("_lio_2", "f64", ee),
        stmt("_lio_3", "f64", ei),
        stmt("_lio_4", "f64", div(mul(ld("taue"), sub(ld("_lio_2"), ld("_lio_1"))), sub(ld("taue"), ld("taum")))),
        stmt("_lio_5", "f64", div(mul(ld("taui"), sub(ld("_lio_3"), ld("_lio_1"))), sub(ld("taui"), ld("taum")))),
        stmt("_lio_6", "f64", sub(ld("El"), mul(ld("El"), ld("_lio_1"))), VOLT),
    ]
    vector = [
        stmt("_v", dtype, n(add(add(add(ld("_lio_6"), mul(ld("_lio_1"), w(ld("v")))),
                                    mul(ld("_lio_4"), w(ld("ge")))), mul(ld("_lio_5"), w(ld("gi"))))),
             VOLT, "not_refractory"),
        stmt("_ge", dtype, n(mul(ld("_lio_2"), w(ld("ge")))), VOLT),
        stmt("_gi", dtype, n(mul(ld("_lio_3"), w(ld("gi")))), VOLT),
        stmt("v", dtype, ld("_v"), VOLT, "not_refractory"),
        stmt("ge", dtype, ld("_ge"), VOLT),
        stmt("gi", dtype, ld("_gi"), VOLT),
    ]
    return scalar, vector


CUBA = dict(taum=20e-3, taue=5e-3, taui=10e-3, Vt=-50e-3, Vr=-60e-3, El=-49e-3,
            we=60 * 0.27 / 10 * 1e-3, wi=-20 * 4.5 / 10 * 1e-3, refractory=5e-3)


def bernoulli_rows(n_source_rows: int, n_target: int, p: float, accept) -> tuple[np.ndarray, np.ndarray]:
    """``Synapses.connect(condition, p)`` with the exporter's draw order (device.py:1032-1048)."""
    sources, targets = [], []
    ids = np.arange(n_target)
    for source in range(n_source_rows):
        selected = np.random.random(n_target) < p
        if accept(source):
            hit = ids[selected]
            sources.append(np.full(hit.size, source, np.int64))
            targets.append(hit)
    return np.concatenate(sources), np.concatenate(targets)


def cuba_network(n: int = 4000, *, exc_fraction: float = 0.8, p: float = 0.02, seed: int = 1729,
                 steps: int = 10000, dt: float = 1e-4, dtype: str = "f32",
                 indegree: int | None = None, weight_scale: float = 1.0, delay_ticks: int = 0,
                 spike_monitor: bool = True, state_monitor: tuple | None = None,
                 event_monitor: list | None = None, poisson_inputs: tuple = (), regular: tuple = (),
                 edge_weights: bool = False) -> dict:
    """CUBA (examples/CUBA.py) as AtlasIR.  ``event_monitor`` lists the variables an
    EventMonitor on the spike event records (at the threshold, before the reset);
    ``poisson_inputs`` = ((target state, N, rate Hz, weight), ...) adds PoissonInputs;
    ``regular`` = ((name, when, statements), ...) adds run_regularly code.

    ``indegree=None`` is config 1: Bernoulli(p) connectivity from the NumPy MT19937
    recipe with ``v0 = Vr + rand()*(Vt - Vr)`` drawn first.  ``indegree=K`` is
    config 3: fixed in-degree K split 80/20 between the excitatory and inhibitory
    source ranges (procedural topology), weights scaled by ``weight_scale``.

    ``edge_weights=True`` (with ``indegree``) gives every synapse its own f32 weight ``w``
    (``ge += w`` / ``gi += w``), drawn by a procedural uniform initializer over
    [0.5, 1.5] times the scaled we or wi, so the mean input is that of the constant weights.
    """
    c = CUBA
    np.random.seed(seed)
    n_exc = int(round(n * exc_fraction))
    v0 = c["Vr"] + np.random.rand(n) * (c["Vt"] - c["Vr"])
    builder = NetworkBuilder(dt=dt, steps=steps, seed=seed)
    zeros = np.zeros(n)
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    w = wide if dtype == "f32" else (lambda e: e)
    nr = narrow if dtype == "f32" else (lambda e: e)
    P = builder.population(
        "neurongroup", n,
        states={"v": (dtype, VOLT, v0), "ge": (dtype, VOLT, zeros), "gi": (dtype, VOLT, zeros)},
        parameters={"taum": scalar(c["taum"], SECOND), "taue": scalar(c["taue"], SECOND),
                    "taui": scalar(c["taui"], SECOND), "El": scalar(c["El"], VOLT),
                    "Vt": scalar(c["Vt"], VOLT), "Vr": scalar(c["Vr"], VOLT)},
        update=cuba_update(dtype),
        threshold=op("gt", w(ld("v")), ld("Vt")),
        reset=[stmt("v", dtype, nr(ld("Vr")), VOLT)],
        refractory=c["refractory"], spike_monitor=spike_monitor, state_monitor=state_monitor,
        event_monitor=event_monitor)
    for target, count, rate, weight in poisson_inputs:
        builder.poisson_input(P, target, count, rate, weight)
    for name, when, statements in regular:
        builder.run_regularly(P, list(statements), when=when, name=name)
    we, wi = c["we"] * weight_scale, c["wi"] * weight_scale
    pre_e = [stmt("ge", dtype, nr(add(w(ld("ge")), ld("we"))), VOLT)]
    pre_i = [stmt("gi", dtype, nr(add(w(ld("gi")), ld("wi"))), VOLT)]
    if indegree is None:
        se, te = bernoulli_rows(n, n, p, lambda i: i < n_exc)
        si, ti = bernoulli_rows(n, n, p, lambda i: i >= n_exc)
        builder.projection("synapses", P, P, on_pre=pre_e, source_range=(0, n), post_aliases={"ge": "ge"},
                           parameters={"we": ("f64", VOLT, we)}, explicit=(se, te), delay_ticks=delay_ticks)
        builder.projection("synapses_1", P, P, on_pre=pre_i, source_range=(0, n), post_aliases={"gi": "gi"},
                           parameters={"wi": ("f64", VOLT, wi)}, explicit=(si, ti), delay_ticks=delay_ticks)
    else:
        k_exc = int(round(indegree * exc_fraction))
        if edge_weights:
            pre_e = [stmt("ge", dtype, nr(add(w(ld("ge")), ld("w"))), VOLT)]
            pre_i = [stmt("gi", dtype, nr(add(w(ld("gi")), ld("w"))), VOLT)]
            params_e = {"w": ("f32", VOLT, None)}
            params_i = {"w": ("f32", VOLT, None)}
            inits_e = {"w": initializer_uniform(0.5 * we, 1.5 * we)}
            inits_i = {"w": initializer_uniform(1.5 * wi, 0.5 * wi)}
        else:
            params_e, params_i = {"we": ("f64", VOLT, we)}, {"wi": ("f64", VOLT, wi)}
            inits_e = inits_i = None
        builder.projection("synapses", P, P, on_pre=pre_e, source_range=(0, n_exc), post_aliases={"ge": "ge"},
                           parameters=params_e, fixed_indegree=k_exc, delay_ticks=delay_ticks,
                           initializers=inits_e)
        builder.projection("synapses_1", P, P, on_pre=pre_i, source_range=(n_exc, n),
                           post_aliases={"gi": "gi"}, parameters=params_i,
                           fixed_indegree=indegree - k_exc, delay_ticks=delay_ticks, initializers=inits_i)
    return builder.document()


def rand(stream: int) -> dict:
    """A uniform draw of the counter RNG (``rand()``) on random stream ``stream``."""
    return {"op": "rand", "stream": int(stream)}


def poisson_network(n_inputs: int = 2000, n: int = 4000, *, rates=(2.0, 40.0), indegree: int = 100,
                    weight: float = 1.0e-3, delay_ticks: int = 1, seed: int = 1729, steps: int = 10000,
                    dt: float = 1e-4, spike_monitor: bool = True) -> dict:
    """A PoissonGroup driving CUBA neurons.

    The PoissonGroup is lowered as the reference exporter lowers it (export.py:1170-1230):
    no state update, threshold ``rand() < rates * dt`` on its own random stream, and rates
    as a per-neuron parameter (uniform in ``rates`` Hz here).  Each CUBA neuron receives
    ``indegree`` distinct Poisson inputs (explicit topology) adding ``weight`` to ``ge``.
    """
    c = CUBA
    rng = np.random.default_rng(seed)
    builder = NetworkBuilder(dt=dt, steps=steps, seed=seed)
    lo, hi = rates
    G = builder.population(
        "poissongroup", n_inputs, states={},
        parameters={"rates": ("f64", (0.0, 0.0, -1.0, 0.0, 0.0, 0.0, 0.0), rng.uniform(lo, hi, n_inputs))},
        threshold=op("lt", rand(0), mul(ld("rates"), ld("dt"))), spike_monitor=spike_monitor)
    v0 = c["Vr"] + rng.random(n) * (c["Vt"] - c["Vr"])
    zeros = np.zeros(n)
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    P = builder.population(
        "neurongroup", n,
        states={"v": ("f32", VOLT, v0), "ge": ("f32", VOLT, zeros), "gi": ("f32", VOLT, zeros)},
        parameters={"taum": scalar(c["taum"], SECOND), "taue": scalar(c["taue"], SECOND),
                    "taui": scalar(c["taui"], SECOND), "El": scalar(-60e-3, VOLT),
                    "Vt": scalar(c["Vt"], VOLT), "Vr": scalar(c["Vr"], VOLT)},
        update=cuba_update("f32"), threshold=op("gt", wide(ld("v")), ld("Vt")),
        reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=c["refractory"], spike_monitor=spike_monitor)
    src, tgt = fixed_indegree_sample(rng, n_inputs, n, indegree)
    builder.projection("synapses", G, P, on_pre=[stmt("ge", "f32", narrow(add(wide(ld("ge")), ld("w"))), VOLT)],
                       post_aliases={"ge": "ge"}, parameters={"w": ("f64", VOLT, weight)}, explicit=(src, tgt),
                       delay_ticks=delay_ticks)
    return builder.document()


def generator_network(n_inputs: int = 500, n: int = 1000, *, spikes: int = 20000, indegree: int = 40,
                      weight: float = 3.0e-3, delay_ticks: int = 1, seed: int = 1729, steps: int = 2000,
                      dt: float = 1e-4) -> dict:
    """A SpikeGeneratorGroup (``spikes`` distinct (tick, neuron) pairs drawn uniformly, plus a
    synchronous volley of every input at tick 10) driving CUBA neurons through ``indegree``
    explicit inputs each adding ``weight`` to ``ge``."""
    c = CUBA
    rng = np.random.default_rng(seed)
    keys = rng.choice(steps * n_inputs, size=min(spikes, steps * n_inputs), replace=False)
    keys = np.union1d(keys, 10 * n_inputs + np.arange(n_inputs))
    builder = NetworkBuilder(dt=dt, steps=steps, seed=seed)
    G = builder.spike_generator("spikegeneratorgroup", n_inputs, keys // n_inputs, keys % n_inputs)
    zeros = np.zeros(n)
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    P = builder.population(
        "neurongroup", n,
        states={"v": ("f32", VOLT, c["Vr"] + rng.random(n) * (c["Vt"] - c["Vr"])), "ge": ("f32", VOLT, zeros),
                "gi": ("f32", VOLT, zeros)},
        parameters={"taum": scalar(c["taum"], SECOND), "taue": scalar(c["taue"], SECOND),
                    "taui": scalar(c["taui"], SECOND), "El": scalar(-60e-3, VOLT),
                    "Vt": scalar(c["Vt"], VOLT), "Vr": scalar(c["Vr"], VOLT)},
        update=cuba_update("f32"), threshold=op("gt", wide(ld("v")), ld("Vt")),
        reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=c["refractory"])
    src, tgt = fixed_indegree_sample(rng, n_inputs, n, indegree)
    builder.projection("synapses", G, P, on_pre=[stmt("ge", "f32", narrow(add(wide(ld("ge")), ld("w"))), VOLT)],
                       post_aliases={"ge": "ge"}, parameters={"w": ("f64", VOLT, weight)}, explicit=(src, tgt),
                       delay_ticks=delay_ticks)
    return builder.document()


def random_pathway_network(n_inputs: int = 300, n: int = 400, *, spikes: int = 3000, indegree: int = 12,
                           draw: str = "rand", procedural: bool = False, cuba: bool = False, stream: int = 1,
                           delay_ticks: int = 1, seed: int = 1729, steps: int = 400, dt: float = 1e-4) -> dict:
    """A SpikeGeneratorGroup (``spikes`` distinct (tick, neuron) pairs and a volley of every input at
    tick 10) driving a population through a pathway that draws from the counter RNG per event,
    indexed by the edge (executor.rs:5071-5074, 5572-5577).

    ``draw`` is "rand" or "randn".  The targets accumulate ``x += draw`` in f64 (no update,
    no threshold), or with ``cuba`` are CUBA neurons with ``ge += w * (0.5 + rand())``.  The
    explicit topology lists its edges in a shuffled order, so that the engine's rows (sorted by
    source and target block) differ from the edge order; ``procedural`` draws a fixed in-degree
    topology instead."""
    c = CUBA
    rng = np.random.default_rng(seed)
    keys = rng.choice(steps * n_inputs, size=min(spikes, steps * n_inputs), replace=False)
    keys = np.union1d(keys, 10 * n_inputs + np.arange(n_inputs))
    builder = NetworkBuilder(dt=dt, steps=steps, seed=seed)
    G = builder.spike_generator("spikegeneratorgroup", n_inputs, keys // n_inputs, keys % n_inputs)
    value = {"op": draw, "stream": int(stream)}
    if cuba:
        zeros = np.zeros(n)
        scalar = lambda v, dims: ("f64", dims, v)  # noqa: E731
        P = builder.population(
            "neurongroup", n,
            states={"v": ("f32", VOLT, c["Vr"] + rng.random(n) * (c["Vt"] - c["Vr"])),
                    "ge": ("f32", VOLT, zeros), "gi": ("f32", VOLT, zeros)},
            parameters={"taum": scalar(c["taum"], SECOND), "taue": scalar(c["taue"], SECOND),
                        "taui": scalar(c["taui"], SECOND), "El": scalar(-60e-3, VOLT),
                        "Vt": scalar(c["Vt"], VOLT), "Vr": scalar(c["Vr"], VOLT)},
            update=cuba_update("f32"), threshold=op("gt", wide(ld("v")), ld("Vt")),
            reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=c["refractory"])
        on_pre = [stmt("ge", "f32", narrow(add(wide(ld("ge")), mul(ld("w"), add(lit(0.5), value)))), VOLT)]
        aliases, params = {"ge": "ge"}, {"w": ("f64", VOLT, 3.0e-3)}
    else:
        P = builder.population("neurongroup", n, states={"x": ("f64", DIMLESS, np.zeros(n))}, frozen=())
        on_pre = [stmt("x", "f64", add(ld("x"), value))]
        aliases, params = {"x": "x"}, None
    if procedural:
        builder.projection("synapses", G, P, on_pre=on_pre, post_aliases=aliases, parameters=params,
                           fixed_indegree=indegree, delay_ticks=delay_ticks)
    else:
        src, tgt = fixed_indegree_sample(rng, n_inputs, n, indegree)
        perm = rng.permutation(src.size)
        builder.projection("synapses", G, P, on_pre=on_pre, post_aliases=aliases, parameters=params,
                           explicit=(src[perm], tgt[perm]), delay_ticks=delay_ticks)
    return builder.document()


def delta_lif_network(n: int = 5000, *, exc_fraction: float = 0.8, indegree: int = 100, seed: int = 1729,
                      steps: int = 2000, dt: float = 1e-4, delays: tuple[int, int] = (2, 1),
                      we: float = 0.2e-3, wi: float = -1.0e-3, dtype: str = "f32") -> dict:
    """LIF with voltage-jump synapses (on_pre ``v += w``), fixed in-degree, two delays.

    dv/dt = (El - v)/taum (unless refractory), El above threshold, v > Vt -> v = Vr,
    refractory 2 ms.  Deliveries and the reset both write ``v``, so the reset must
    run after the tick's deliveries (it cannot be fused with the update).
    """
    np.random.seed(seed)
    taum, El, Vt, Vr = 20e-3, -48e-3, -50e-3, -60e-3
    n_exc = int(round(n * exc_fraction))
    v0 = Vr + np.random.rand(n) * (Vt - Vr)
    builder = NetworkBuilder(dt=dt, steps=steps, seed=seed)
    w = wide if dtype == "f32" else (lambda e: e)
    nr = narrow if dtype == "f32" else (lambda e: e)
    scalar = [stmt("_lio_1", "f64", un("exp", div(neg(ld("dt")), ld("taum"))))]
    vector = [stmt("_v", dtype, nr(add(ld("El"), mul(sub(w(ld("v")), ld("El")), ld("_lio_1")))), VOLT,
                   "not_refractory"),
              stmt("v", dtype, ld("_v"), VOLT, "not_refractory")]
    P = builder.population(
        "neurongroup", n, states={"v": (dtype, VOLT, v0)},
        parameters={"taum": ("f64", SECOND, taum), "El": ("f64", VOLT, El), "Vt": ("f64", VOLT, Vt),
                    "Vr": ("f64", VOLT, Vr)},
        update=(scalar, vector), threshold=op("gt", w(ld("v")), ld("Vt")),
        reset=[stmt("v", dtype, nr(ld("Vr")), VOLT)], refractory=2e-3)
    k_exc = int(round(indegree * exc_fraction))
    builder.projection("exc", P, P, on_pre=[stmt("v", dtype, nr(add(w(ld("v")), ld("we"))), VOLT)],
                       source_range=(0, n_exc), post_aliases={"v": "v"},
                       parameters={"we": ("f64", VOLT, we)}, fixed_indegree=k_exc, delay_ticks=delays[0])
    builder.projection("inh", P, P, on_pre=[stmt("v", dtype, nr(add(w(ld("v")), ld("wi"))), VOLT)],
                       source_range=(n_exc, n), post_aliases={"v": "v"},
                       parameters={"wi": ("f64", VOLT, wi)}, fixed_indegree=indegree - k_exc,
                       delay_ticks=delays[1])
    return builder.document()


# ------------------------------------------------------------------- COBAHH family
COBAHH = dict(area=20000e-12, El=-60e-3, EK=-90e-3, ENa=50e-3, VT=-63e-3, taue=5e-3, taui=10e-3, Ee=0.0,
              Ei=-80e-3, we=6e-9, wi=67e-9, refractory=3e-3, threshold=-20e-3)
COBAHH.update(Cm=1e-2 * COBAHH["area"], gl=5e-5 * 1e4 * COBAHH["area"], g_na=100e-3 * 1e4 * COBAHH["area"],
              g_kd=30e-3 * 1e4 * COBAHH["area"])


def hh_update(dtype: str = "f32", external_current: bool = False) -> tuple[list, list]:
    """Exponential-Euler update of the Hodgkin-Huxley equations of examples/COBAHH.py:37-53.

    Each state x with dx/dt = A + B x advances as x' = -A/B + (x + A/B) exp(B dt),
    every right-hand side reading the start-of-tick states (Brian2's
    ``exponential_euler``).  Rates in SI units:
      alpha_m = 1280/exprel((13 mV - v + VT)/4 mV),  beta_m = 1400/exprel((v - VT - 40 mV)/5 mV),
      alpha_h = 128 exp((17 mV - v + VT)/18 mV),     beta_h = 4000/(1 + exp((40 mV - v + VT)/5 mV)),
      alpha_n = 160/exprel((15 mV - v + VT)/5 mV),   beta_n = 500 exp((10 mV - v + VT)/40 mV).
    ``external_current`` adds a per-neuron constant current I_ext to dv/dt (the
    reference's gpu_hh.py workload).  The ODEs are not gated by refractoriness.
    """
    w = wide if dtype == "f32" else (lambda e: e)
    n_ = narrow if dtype == "f32" else (lambda e: e)
    v, m, h, nn, ge, gi = (w(ld(x)) for x in ("v", "m", "h", "n", "ge", "gi"))
    mv = lambda x: lit(x * 1e-3)  # noqa: E731
    er = lambda x: un("exprel", x)  # noqa: E731
    ex = lambda x: un("exp", x)  # noqa: E731
    rates = {
        "m": (div(lit(1280.0), er(div(add(sub(mv(13), v), ld("VT")), mv(4)))),
              div(lit(1400.0), er(div(sub(sub(v, ld("VT")), mv(40)), mv(5))))),
        "h": (mul(lit(128.0), ex(div(add(sub(mv(17), v), ld("VT")), mv(18)))),
              div(lit(4000.0), add(lit(1.0), ex(div(add(sub(mv(40), v), ld("VT")), mv(5)))))),
        "n": (div(lit(160.0), er(div(add(sub(mv(15), v), ld("VT")), mv(5)))),
              mul(lit(500.0), ex(div(add(sub(mv(10), v), ld("VT")), mv(40))))),
    }
    vector = []
    for x in ("m", "n", "h"):
        alpha, beta = rates[x]
        vector += [stmt(f"_alpha_{x}", "f64", alpha), stmt(f"_beta_{x}", "f64", beta),
                   stmt(f"_B_{x}", "f64", neg(add(ld(f"_alpha_{x}"), ld(f"_beta_{x}")))),
                   stmt(f"_BA_{x}", "f64", div(ld(f"_alpha_{x}"), ld(f"_B_{x}"))),
                   stmt(f"_{x}", dtype, n_(add(neg(ld(f"_BA_{x}")),
                                               mul(add(ld(f"_BA_{x}"), w(ld(x))), ex(mul(ld(f"_B_{x}"), ld("dt"))))))),
                   ]
    gna = mul(mul(ld("g_na"), mul(mul(m, m), m)), h)
    gk = mul(ld("g_kd"), mul(mul(nn, nn), mul(nn, nn)))
    vector += [stmt("_gna", "f64", gna, SIEMENS), stmt("_gk", "f64", gk, SIEMENS),
               stmt("_gsum", "f64", add(add(add(add(ld("gl"), ge), gi), ld("_gna")), ld("_gk")), SIEMENS)]
    drive = add(add(add(add(mul(ld("gl"), ld("El")), mul(ge, ld("Ee"))), mul(gi, ld("Ei"))),
                    mul(ld("_gna"), ld("ENa"))), mul(ld("_gk"), ld("EK")))
    if external_current:
        drive = add(drive, w(ld("I_ext")))
    vector += [stmt("_B_v", "f64", div(neg(ld("_gsum")), ld("Cm"))),
               stmt("_BA_v", "f64", div(neg(drive), ld("_gsum")), VOLT),
               stmt("_v", dtype, n_(add(neg(ld("_BA_v")), mul(add(ld("_BA_v"), v), ex(mul(ld("_B_v"), ld("dt")))))),
                    VOLT),
               stmt("_ge", dtype, n_(mul(ge, ex(div(neg(ld("dt")), ld("taue"))))), SIEMENS),
               stmt("_gi", dtype, n_(mul(gi, ex(div(neg(ld("dt")), ld("taui"))))), SIEMENS)]
    for x, dims in (("m", DIMLESS), ("n", DIMLESS), ("h", DIMLESS), ("v", VOLT), ("ge", SIEMENS), ("gi", SIEMENS)):
        vector.append(stmt(x, dtype, ld(f"_{x}"), dims))
    return [], vector


def _hh_parameters() -> dict:
    c = COBAHH
    s = lambda value, dims: ("f64", dims, value)  # noqa: E731
    return {"Cm": s(c["Cm"], FARAD), "gl": s(c["gl"], SIEMENS), "g_na": s(c["g_na"], SIEMENS),
            "g_kd": s(c["g_kd"], SIEMENS), "El": s(c["El"], VOLT), "EK": s(c["EK"], VOLT), "ENa": s(c["ENa"], VOLT),
            "VT": s(c["VT"], VOLT), "Ee": s(c["Ee"], VOLT), "Ei": s(c["Ei"], VOLT), "taue": s(c["taue"], SECOND),
            "taui": s(c["taui"], SECOND)}


def cobahh_network(n: int = 4000, *, exc_fraction: float = 0.8, p: float = 0.02, seed: int = 1729,
                   steps: int = 10000, dt: float = 1e-4, dtype: str = "f32", delay_ticks: int = 0,
                   spike_monitor: bool = True) -> dict:
    """COBAHH (examples/COBAHH.py) as AtlasIR: HH neurons, exponential-Euler update,
    threshold v > -20 mV, refractory 3 ms, no reset; Pe -> P ``ge += we`` (6 nS) and
    Pi -> P ``gi += wi`` (67 nS), Bernoulli p.  NumPy MT19937 replay of the script's
    order: both connect() calls, then v = El + (randn()*5 - 5) mV,
    ge = (randn()*1.5 + 4)*10 nS, gi = (randn()*12 + 20)*10 nS; m = n = h = 0."""
    c = COBAHH
    np.random.seed(seed)
    n_exc = int(round(n * exc_fraction))
    se, te = bernoulli_rows(n_exc, n, p, lambda i: True)
    si, ti = bernoulli_rows(n - n_exc, n, p, lambda i: True)
    v0 = c["El"] + (np.random.randn(n) * 5 - 5) * 1e-3
    ge0 = (np.random.randn(n) * 1.5 + 4) * 10e-9
    gi0 = (np.random.randn(n) * 12 + 20) * 10e-9
    zeros = np.zeros(n)
    builder = NetworkBuilder(dt=dt, steps=steps, seed=seed)
    w = wide if dtype == "f32" else (lambda e: e)
    nr = narrow if dtype == "f32" else (lambda e: e)
    P = builder.population(
        "neurongroup", n,
        states={"v": (dtype, VOLT, v0), "m": (dtype, DIMLESS, zeros), "n": (dtype, DIMLESS, zeros),
                "h": (dtype, DIMLESS, zeros), "ge": (dtype, SIEMENS, ge0), "gi": (dtype, SIEMENS, gi0)},
        parameters=_hh_parameters(), update=hh_update(dtype),
        threshold=op("gt", w(ld("v")), lit(c["threshold"])), refractory=c["refractory"], frozen=(),
        spike_monitor=spike_monitor)
    builder.projection("synapses", P, P, on_pre=[stmt("ge", dtype, nr(add(w(ld("ge")), ld("we"))), SIEMENS)],
                       source_range=(0, n_exc), post_aliases={"ge": "ge"},
                       parameters={"we": ("f64", SIEMENS, c["we"])}, explicit=(se, te), delay_ticks=delay_ticks)
    builder.projection("synapses_1", P, P, on_pre=[stmt("gi", dtype, nr(add(w(ld("gi")), ld("wi"))), SIEMENS)],
                       source_range=(n_exc, n), post_aliases={"gi": "gi"},
                       parameters={"wi": ("f64", SIEMENS, c["wi"])}, explicit=(si, ti), delay_ticks=delay_ticks)
    return builder.document()


# ------------------------------------------------------------ plastic network
def fixed_indegree_sample(rng: np.random.Generator, n_src: int, n_tgt: int, k: int) -> tuple[np.ndarray, np.ndarray]:
    """k distinct sources per target, drawn uniformly (draws that repeat a source of the same
    target are redrawn until none repeats); returned source-major, targets ascending."""
    if k > n_src:
        raise ValueError("in-degree exceeds the source count")
    x = rng.integers(0, n_src, (n_tgt, k), dtype=np.int64)
    while True:
        x.sort(axis=1)
        repeat = np.zeros(x.shape, bool)
        repeat[:, 1:] = x[:, 1:] == x[:, :-1]
        count = int(repeat.sum())
        if not count:
            break
        x[repeat] = rng.integers(0, n_src, count, dtype=np.int64)
    sources = x.reshape(-1)
    targets = np.repeat(np.arange(n_tgt, dtype=np.int64), k)
    order = np.argsort(sources, kind="stable")
    return sources[order], targets[order]


def plastic_network(n: int = 100_000, *, exc_fraction: float = 0.8, indegree: int = 1000, delays: tuple = (1, 20),
                    steps: int = 100_000, dt: float = 1e-4, seed: int = 1729, wmax: float = 2e-3,
                    we: float = 1e-3, wi: float = -3.5e-3, taupre: float = 20e-3, taupost: float = 20e-3,
                    apre: float = 0.01, apost: float = -0.0105, packed: bool = True,
                    spike_monitor: bool = True) -> dict:
    """Config 5: plastic, delayed CUBA LIF network.

    CUBA neurons (examples/CUBA.py dynamics, refractory 5 ms); fixed in-degree
    ``indegree`` split 80/20 between excitatory and inhibitory sources, explicit
    topology (synapse states need one); per-synapse delays uniform in
    ``delays`` ticks.  Excitatory -> excitatory synapses carry pair-based STDP
    (examples/synapses/STDP.py:33-42 with event-driven traces, synapses.py:359-383):
    w (float32, volts) clipped to [0, wmax], w0 ~ U[0, wmax], traces with
    taupre = taupost = 20 ms, increments apre * wmax and apost * wmax; on_pre adds w
    to ge.  Excitatory -> inhibitory synapses add ``we`` to ge, inhibitory synapses
    add ``wi`` to gi.  ``packed`` keeps the 1e8-edge arrays as numpy.
    """
    c = CUBA
    rng = np.random.default_rng(seed)
    n_exc = int(round(n * exc_fraction))
    k_exc = int(round(indegree * exc_fraction))
    builder = NetworkBuilder(dt=dt, steps=steps, seed=seed, packed=packed)
    v0 = c["Vr"] + rng.random(n) * (c["Vt"] - c["Vr"])
    zeros = np.zeros(n)
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    P = builder.population(
        "neurongroup", n,
        states={"v": ("f32", VOLT, v0), "ge": ("f32", VOLT, zeros), "gi": ("f32", VOLT, zeros)},
        parameters={"taum": scalar(c["taum"], SECOND), "taue": scalar(c["taue"], SECOND),
                    "taui": scalar(c["taui"], SECOND), "El": scalar(c["El"], VOLT),
                    "Vt": scalar(c["Vt"], VOLT), "Vr": scalar(c["Vr"], VOLT)},
        update=cuba_update("f32"), threshold=op("gt", wide(ld("v")), ld("Vt")),
        reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=c["refractory"], spike_monitor=spike_monitor)
    lo, hi = delays
    # excitatory -> excitatory, plastic
    src, tgt = fixed_indegree_sample(rng, n_exc, n_exc, k_exc)
    e = src.size
    elapsed = sub(ld("t"), ld("lastupdate"))
    decay = [stmt("Apre", "f32", narrow(mul(wide(ld("Apre")), un("exp", div(neg(elapsed), ld("taupre")))))),
             stmt("Apost", "f32", narrow(mul(wide(ld("Apost")), un("exp", div(neg(elapsed), ld("taupost"))))))]
    clip = lambda x: {"op": "clip", "value": x, "min": lit(0.0), "max": ld("wmax")}  # noqa: E731
    on_pre = decay + [stmt("ge", "f32", narrow(add(wide(ld("ge")), wide(ld("w")))), VOLT),
                      stmt("Apre", "f32", narrow(add(wide(ld("Apre")), ld("dApre")))),
                      stmt("w", "f32", narrow(clip(add(wide(ld("w")), wide(ld("Apost"))))), VOLT),
                      stmt("lastupdate", "f64", ld("t"), SECOND)]
    on_post = decay + [stmt("Apost", "f32", narrow(add(wide(ld("Apost")), ld("dApost")))),
                       stmt("w", "f32", narrow(clip(add(wide(ld("w")), wide(ld("Apre"))))), VOLT),
                       stmt("lastupdate", "f64", ld("t"), SECOND)]
    builder.projection(
        "synapses", P, P, on_pre=on_pre, on_post=on_post, source_range=(0, n_exc), target_range=(0, n_exc),
        post_aliases={"ge": "ge"},
        states={"w": ("f32", VOLT, rng.uniform(0.0, wmax, e).astype(np.float32)),
                "Apre": ("f32", DIMLESS, np.zeros(e, np.float32)), "Apost": ("f32", DIMLESS, np.zeros(e, np.float32)),
                "lastupdate": ("f64", SECOND, np.zeros(e))},
        parameters={"taupre": scalar(taupre, SECOND), "taupost": scalar(taupost, SECOND),
                    "wmax": scalar(wmax, VOLT), "dApre": scalar(apre * wmax, VOLT),
                    "dApost": scalar(apost * wmax, VOLT)},
        explicit=(src, tgt), delay_ticks=rng.integers(lo, hi + 1, e))
    del src, tgt
    # excitatory -> inhibitory, static
    src, tgt = fixed_indegree_sample(rng, n_exc, n - n_exc, k_exc)
    builder.projection("synapses_1", P, P, on_pre=[stmt("ge", "f32", narrow(add(wide(ld("ge")), ld("we"))), VOLT)],
                       source_range=(0, n_exc), target_range=(n_exc, n), post_aliases={"ge": "ge"},
                       parameters={"we": scalar(we, VOLT)}, explicit=(src, tgt),
                       delay_ticks=rng.integers(lo, hi + 1, src.size))
    del src, tgt
    # inhibitory -> all, static
    src, tgt = fixed_indegree_sample(rng, n - n_exc, n, indegree - k_exc)
    builder.projection("synapses_2", P, P, on_pre=[stmt("gi", "f32", narrow(add(wide(ld("gi")), ld("wi"))), VOLT)],
                       source_range=(n_exc, n), post_aliases={"gi": "gi"}, parameters={"wi": scalar(wi, VOLT)},
                       explicit=(src, tgt), delay_ticks=rng.integers(lo, hi + 1, src.size))
    return builder.document()


def with_recording_window(document: dict, window_steps: int) -> dict:
    """The sealed document with every population's monitors bounded to its last `window_steps`
    ticks, as the reference Device's ``recording_window_steps`` option lowers it (the window is
    min(steps, window_steps), export.py:724-725): state samples, the spike monitor (ticks and
    counts) and the spike event stream keep only the ticks at or after end - window
    (executor.rs:2993, 3038-3051, 3082-3087)."""
    if not 1 <= int(window_steps) <= 10_000_000:
        raise ValueError("recording_window_steps must be an integer within 1..10,000,000")
    doc = protocol.load(document, verify_envelope=False)
    doc.pop("protocol", None)
    for pdef in doc["definition"]["populations"]:
        pdef["monitor"]["window_steps"] = min(int(pdef["steps"]), int(window_steps))
    return protocol.seal(doc)


def to_binary_csr(document: dict, synapse: int, path) -> dict:
    """The document with an explicit-topology Synapses' edges moved to a B2CSR001 file at
    `path`, as ``connect_binary_csr`` declares them (python/brian2_rust/__init__.py:35-40,
    topology kind ``binary_csr``): edges source-major, each per-edge parameter (f64) one
    column.  The edges are sorted by source stably, so every target still receives a
    source's events in edge order after the events of lower sources: the canonical
    delivery order, hence the results, are unchanged."""
    import copy
    from . import binary_topology
    from .engine import decode_array
    doc = copy.deepcopy(protocol.load(document, verify_envelope=False))
    doc.pop("protocol", None)
    sdef, sin = doc["definition"]["synapses"][synapse], doc["instance"]["synapses"][synapse]
    src = np.asarray(sin["source"], np.int64)
    tgt = np.asarray(sin["target"], np.int64)
    order = np.argsort(src, kind="stable")
    offsets = np.zeros(sdef["source_count"] + 1, np.int64)
    np.cumsum(np.bincount(src, minlength=sdef["source_count"]), out=offsets[1:])
    names = [p["name"] for p in sdef["parameters"] if p["index_domain"] == "synapse"]
    columns = [decode_array(sin["parameters"][name], "f64")[order] for name in names]
    sha = binary_topology.write_csr(path, sdef["source_count"], sdef["target_count"], offsets, tgt[order], columns)
    for name in names:
        sin["parameters"][name] = []
    sin["source"], sin["target"] = [], []
    sin["topology"] = {"kind": "binary_csr", "edge_count": int(src.size), "path": str(path), "sha256": sha,
                       "column_count": len(names), "initializers": {name: k for k, name in enumerate(names)}}
    return protocol.seal(doc)


def binary_csr_example(dt: float = 1e-4, steps: int = 20) -> tuple[dict, tuple]:
    """The reference's B2CSR001 conformance model (tests/test_binary_topology.py:19-98):
    four neurons ``dv/dt = (1.2 - v) / (10 ms)`` (Euler), threshold ``v > 1``, reset
    ``v = 0``, v0 = linspace(0, 1.1, 4); Synapses with a constant per-edge
    ``multiplicity``, on_pre ``v_post += 0.02 * multiplicity``, delay 0.2 ms; the
    fixture graph offsets [0, 2, 3, 4, 5], targets [0, 2, 3, 1, 0], multiplicity
    [1, 3, 2, 4, 5]; 2 ms.  Returns the explicit-topology document and the CSR arrays
    (offsets, targets, multiplicity) for ``to_binary_csr``."""
    offsets = np.array([0, 2, 3, 4, 5])
    targets = np.array([0, 2, 3, 1, 0])
    multiplicity = np.array([1.0, 3.0, 2.0, 4.0, 5.0])
    builder = NetworkBuilder(dt=dt, steps=steps, seed=0)
    tau = 10e-3
    # Euler: v <- v + dt * (1.2 - v) / tau, in f64
    update = ([], [stmt("v", "f64", add(ld("v"), mul(ld("dt"), div(sub(lit(1.2), ld("v")), ld("tau")))))])
    pop = builder.population(
        "neurons", 4, states={"v": ("f64", DIMLESS, np.linspace(0.0, 1.1, 4))},
        parameters={"tau": ("f64", SECOND, tau)}, update=update, threshold=op("gt", ld("v"), lit(1.0)),
        reset=[stmt("v", "f64", lit(0.0))], spike_monitor=True, state_monitor=(["v"], [0, 1, 2, 3]))
    builder.projection(
        "projection", pop, pop, on_pre=[stmt("v", "f64", add(ld("v"), mul(lit(0.02), ld("multiplicity"))))],
        post_aliases={"v": "v"}, parameters={"multiplicity": ("f64", DIMLESS, multiplicity)},
        explicit=(np.repeat(np.arange(4), np.diff(offsets)), targets), delay_ticks=2)
    return builder.document(), (offsets, targets, multiplicity)

