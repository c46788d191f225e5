"""``HipExecutor``: the MI355X replacement of the reference ``CudaExecutor``.

Constructor keywords and the result dictionary mirror ``CudaExecutor``
(brian2-rust/python/brian2_rust/cuda.py:80-392) and ``run_dag``
(metal_dag.py:589-652): ``run()`` returns ``{populations, synapses,
numeric_profile, device, timings, run_seconds, compile_seconds, plan_sha256,
rng_profile, hip_runtime}`` with per-population ``states, trace, spike_ticks,
indices, counts, last_spikes, refractory, event_streams`` (each stream a
``dict(ticks=, indices=)``, metal_dag.py:624-628) and per-synapse ``states,
events``.  ``timings`` is the reference's list of ``{input_seconds,
command_seconds, gpu_seconds, readback_seconds}`` (metal_dag.py:645), which the
reference result writer sums (metal.py:1003-1004).  ``rng_profile`` is ``None``
for a model without random draws, as the writer requires (metal.py:929); a model
with ``rand``/``randn``/``binomial``/``poisson`` draws reports the document's
``rng_algorithm`` (``splitmix64-counter-v1``): the engine draws the reference CPU
engine's f64 counter values (executor.rs:190-323), not the reference GPU's
24-bit float32 profile ``b2-counter-f32-u24-v0``.

Execution is one hiprtc module per model (atlas_hip.engine) driven by the
native runtime (libatlas_sim_hip.so).  Each ``run()`` replays the initial
snapshot, as the reference executor does.  Numeric faults raise
``FloatingPointError``; the reference's 10,000,000 recorded events per stream
limit (executor.rs:2993-2998) raises ``RuntimeError`` unless lifted.
"""
from __future__ import annotations

import os
import time
from pathlib import Path

import numpy as np

from . import engine, native
from .engine import NUMPY

RECORDING_BUDGET = 10_000_000
NUMERIC_PROFILE = "reference-f64-registers/f32-storage-hip-v1"
QUEUE_OVERFLOW = 8   # fault bit: a delivery queue dropped records (atlas_tick.h ATLAS_FAULT_QUEUE)
RING_STALL = 32      # fault bit: a persistent launch's wait for a ring word ran out (ATLAS_FAULT_STALL)
EDGE_NODES = 64      # fault bit: the split loop's edge-keyed lists ran out of nodes (ATLAS_FAULT_EDGES)
RING_VALUE = 0xFFFFF # value bits of a persistent launch's stamped ring words (ATLAS_RING_VALUE)
RANDOM_OPS = frozenset({"rand", "randn", "binomial", "poisson"})


class PlanValidationError(ValueError):
    """An executor option the HIP engine does not implement (the reference's
    PlanValidationError, cuda.py:60-61, 91-92)."""


def has_random(value) -> bool:
    """Whether an AtlasIR definition draws random numbers (the reference's RANDOM_OPS test,
    metal_random.py:10-16)."""
    if isinstance(value, dict):
        return value.get("op") in RANDOM_OPS or any(has_random(v) for v in value.values())
    return isinstance(value, (list, tuple)) and any(has_random(v) for v in value)


class HipExecutor:
    """Compile once, then replay the initial snapshot on one MI355X device."""

    def __init__(self, model, directory=None, *, numeric_mode="float32", runner=None, plan=None,
                 event_delivery="scan", dag_execution="auto", compile_reuse=False, reuse_from=None,
                 synapse_prefix=False, synapse_fusion=False, synapse_sparse=False, device=None,
                 lift_recording_budget=False, verify_envelope=True, shape=None):
        if numeric_mode != "float32":
            # the engine stores states in their declared dtypes with f64 registers, the only mode it has
            raise PlanValidationError("the HIP executor supports numeric_mode='float32' only")
        if plan is not None:
            raise PlanValidationError("the HIP executor lowers the model itself; a prebuilt plan is not accepted")
        del runner, event_delivery, dag_execution, reuse_from, synapse_prefix, synapse_fusion, synapse_sparse
        self.closed = True
        self.directory = Path(directory) if directory is not None else None
        self.lift_recording_budget = lift_recording_budget
        started = time.perf_counter()
        self.plan = engine.lower(model, verify_envelope=verify_envelope, shape=shape)
        self.document = self.plan.document
        engine.allocate(self.plan)
        engine.generate(self.plan, native.device_header_text())
        self.sim = native.Sim(device)
        self.closed = False
        self._dynamic = []
        for index, buffer in enumerate(self.plan.buffers):
            got = self.sim.alloc(buffer.nbytes, buffer.init)
            if got != index:
                raise RuntimeError("device buffer table out of order")
        self._dynamic = [k for k, b in enumerate(self.plan.buffers) if self._is_dynamic(b.name)]
        # pristine device copies of initialised mutable buffers: replays restore on the device
        self._pristine = {k: self.sim.alloc(self.plan.buffers[k].nbytes, self.plan.buffers[k].init)
                          for k in self._dynamic if self.plan.buffers[k].init is not None}
        self._build_topologies()
        if self._build_slots():
            engine.generate(self.plan, native.device_header_text())
        lowered = time.perf_counter()
        # persistent launches (one cooperative launch for many ticks, states in registers) where the
        # plan allows them; ATLAS_HIP_PERSISTENT=0 keeps one launch per tick, =plain issues them as
        # ordinary launches once the kernel's occupancy shows the grid fits (for kernel tracers
        # that cannot follow cooperative launches)
        mode = os.environ.get("ATLAS_HIP_PERSISTENT", "1")
        self.persistent = mode != "0"
        self.plain_launches = mode == "plain"
        self._compile()
        self.compile_seconds = time.perf_counter() - lowered
        self.setup_seconds = lowered - started
        self.compilation_report = dict(requested=compile_reuse, kernels_compiled=len(self.plan.kernels),
                                       kernels_reused=0, source_bytes=len(self.plan.source),
                                       compiler_options=list(engine.COMPILE_OPTIONS))
        self.device_name = self.sim.device_name()
        self.random = has_random(self.document["definition"])
        self._fresh = True

    def _compile(self) -> None:
        """Compile the plan's module and set its launches: the per-tick schedule and epilogue, and
        the persistent launch when the plan has one and persistent launches are enabled."""
        self.sim.compile(self.plan.source, self.plan.kernels, engine.COMPILE_OPTIONS)
        self.sim.set_schedule(self.plan.launches)
        self.sim.set_epilogue(self.plan.epilogue)
        try:
            self.sim.set_persistent(self.plan.persistent if self.persistent else None, self.plan.barrier_buffer,
                                    engine.PERSISTENT_TICKS, plain=self.plain_launches)
        except native.NativeError as error:
            if error.code != native.COOPERATIVE:
                raise
            self.persistent = False   # the grid cannot be resident at once: one launch per tick
            self.sim.set_persistent(None)

    @property
    def launch_mode(self) -> str:
        return "persistent" if self.persistent and self.plan.persistent is not None else "per-tick"

    def _run_ticks(self, steps: int):
        """The tick loop; a persistent grid the device cannot hold at once (nothing ran) falls back to
        one launch per tick for the rest of the executor's life."""
        try:
            return self.sim.run(self.plan.start_tick, steps)
        except native.NativeError as error:
            if error.code != native.COOPERATIVE:
                raise
        self.persistent = False
        self.sim.set_persistent(None)
        self.reset()
        return self.sim.run(self.plan.start_tick, steps)

    @staticmethod
    def _is_dynamic(name: str) -> bool:
        # tables built once, and queue records (only read below their counters)
        static = (".param.", ".row_target", ".segment", ".slots", ".monitor_entries", ".monitor_offsets",
                  ".queue_records", ".queue_scratch", ".generator_offsets", ".generator_ticks", ".records",
                  ".pending", ".refractory_table", "clock_table")
        return not any(part in name for part in static)

    def _build_topologies(self) -> None:
        for path in self.plan.pathways:
            if path.topology[0] != "fixed_indegree":
                continue
            _, indegree, seed = path.topology
            tpop = self.plan.populations[path.target]
            spec = native.FixedIndegree(
                source_count=path.scount, target_count=path.tcount, indegree=indegree, seed=seed,
                target_start=path.tstart, block=self.plan.shape.block, blocks=tpop.blocks,
                row_target_buffer=path.buffers["row_tgt"], segment_buffer=path.buffers["seg"])
            self.sim.fixed_indegree(spec)

    def _build_slots(self) -> bool:
        """Fill the slot tables of counting groups from their segment and row tables (segments
        above engine.SLOT_TARGETS events keep their first row in the slot); a pathway with a
        segment above engine.SLOT_MAX_COUNT events puts its group back on the row-table
        delivery.  Returns whether the module must be regenerated."""
        fallback = False
        for path in self.plan.pathways:
            if "slot" not in path.buffers:
                continue
            tpop = self.plan.populations[path.target]
            spec = native.SlotTable(
                segment_buffer=path.buffers["seg"], row_target_buffer=path.buffers["row_tgt"],
                slot_buffer=path.buffers["slot"], block=self.plan.shape.block, groups=path.scount * len(path.dvals),
                blocks=tpop.blocks, first_block=tpop.first_block, per_xcd=engine.per_xcd(self.plan),
                xcds=engine.XCDS, row_slots=int(path.row_slots))
            largest = self.sim.build_slots(spec)
            if largest > engine.SLOT_MAX_COUNT:
                self.plan.slot_fallback.add(path.index)
                fallback = True
        return fallback

    def _enlarge_queues(self) -> None:
        """Grow every queued group's records per (arrival slot, target block) fourfold, up to
        the exact bound (its in-edges per block), then recompile against the new buffers.
        The old record buffers stay allocated until close."""
        grown = False
        for group in self.plan.groups:
            info = self.plan.queues.get(group[0].index)
            if info is None or info["cap"] >= info["limit"]:
                continue
            info["cap"] = min(info["limit"], info["cap"] * 4)
            blocks = self.plan.populations[group[0].target].blocks
            group[0].buffers["queue"] = self.sim.alloc(info["depth"] * blocks * info["cap"] * 8)
            group[0].buffers["queue_scratch"] = self.sim.alloc(blocks * info["cap"] * 8)
            grown = True
        if not grown:
            raise RuntimeError("delivery queue overflow at its exact bound")
        engine.generate(self.plan, native.device_header_text())
        self._compile()

    # ------------------------------------------------------------------ run
    def reset(self) -> None:
        """Restore the initial snapshot of every mutable buffer."""
        for k in self._dynamic:
            if k in self._pristine:
                self.sim.copy(k, self._pristine[k], self.plan.buffers[k].nbytes)
            else:
                self.sim.zero(k)

    def run(self, *, max_buffer_bytes=None, compute="gpu", workers=None, dag_execution=None,
            ticks: int | None = None, profile: bool = False, collect: bool = True) -> dict:
        if self.closed:
            raise RuntimeError("executor is closed")
        if compute != "gpu":
            raise ValueError("the HIP executor only computes on the GPU")
        del max_buffer_bytes, workers, dag_execution
        started = time.perf_counter()
        if not self._fresh:
            self.reset()
        self._fresh = False
        plan = self.plan
        steps = plan.steps if ticks is None else int(ticks)
        if not 0 <= steps <= plan.steps:
            raise ValueError(f"ticks must lie in [0, {plan.steps}]")
        self.sim.set_profiling(profile)
        command_started = time.perf_counter()
        input_seconds = command_started - started
        stats = self._run_ticks(steps)
        fault = self.sim.read(plan.fault_buffer, np.uint32, 4)
        while fault[0] & QUEUE_OVERFLOW:
            # a delivery queue overflowed (its records were dropped): enlarge and replay
            self._enlarge_queues()
            self.reset()
            stats = self._run_ticks(steps)
            fault = self.sim.read(plan.fault_buffer, np.uint32, 4)
        if fault[0] & EDGE_NODES and self.launch_mode == "persistent":
            # a tick listed more events into one block than its LDS holds (events were dropped):
            # replay with one launch per tick, whose ordered delivery stages events in windows,
            # for the rest of the executor's life
            self.persistent = False
            self.sim.set_persistent(None)
            self.reset()
            stats = self._run_ticks(steps)
            fault = self.sim.read(plan.fault_buffer, np.uint32, 4)
        if fault[0] & RING_STALL:
            raise RuntimeError("a persistent launch's wait for the spike ring timed out; its results are invalid")
        command_seconds = time.perf_counter() - command_started
        self.last_stats = stats
        self.kernel_times = {name: self.sim.kernel_time(k) for k, name in enumerate(plan.kernels)} if profile else {}
        if fault[0]:
            reasons = []
            if fault[0] & 1:
                reasons.append("non-finite numeric value")
            if fault[0] & 2:
                reasons.append("timestep outside Brian2 int64 range")
            if fault[0] & 4:
                reasons.append("refractory deadline search did not converge")
            if fault[0] & 16:
                reasons.append("invalid binomial probability")
            raise FloatingPointError("GPU numeric evaluation failed: " + ", ".join(reasons))
        runtime = {"device_seconds": stats.device_seconds, "host_seconds": stats.host_seconds,
                   "launches": int(stats.launches), "ticks": steps, "architecture": "gfx950",
                   "launch_mode": self.launch_mode,
                   "timing_scope": "HIP-event interval of the tick launches on the library's stream"}
        if not collect:
            return {"timings": [self._timing(input_seconds, command_seconds, stats, 0.0)], "hip_runtime": runtime,
                    "ticks": steps}
        readback_started = time.perf_counter()
        result = self._collect(steps)
        result["timings"] = [self._timing(input_seconds, command_seconds, stats,
                                          time.perf_counter() - readback_started)]
        result["hip_runtime"] = runtime
        result["run_seconds"] = time.perf_counter() - started
        result["compile_seconds"] = self.compile_seconds
        result["plan_sha256"] = plan.sha256
        result["rng_profile"] = self.document["definition"].get("rng_algorithm", "splitmix64-counter-v1") \
            if self.random else None
        result["numeric_profile"] = NUMERIC_PROFILE
        result["device"] = self.device_name
        return result

    @staticmethod
    def _timing(input_seconds: float, command_seconds: float, stats, readback_seconds: float) -> dict:
        """One entry of the reference's ``timings`` list (metal_dag.py:645): snapshot restore,
        the simulation command (host wall time of the tick loop, overflow replays included), its
        device time, and the result read-back."""
        return {"input_seconds": input_seconds, "command_seconds": command_seconds,
                "gpu_seconds": stats.device_seconds, "readback_seconds": readback_seconds}

    def _collect(self, steps: int) -> dict:
        plan = self.plan
        populations = []
        for pop in plan.populations:
            b = pop.buffers
            # with several clocks each population has advanced its own clock's ticks
            end_tick = plan.end_tick(pop, steps)
            last_tick = end_tick - 1
            ran = end_tick > pop.start_tick
            states = {name: self.sim.read(b[f"state:{name}"], NUMPY[dtype], pop.count)
                      for name, dtype, _ in pop.states}
            rows = max(0, end_tick - pop.window_start)
            if pop.has_spike_event and rows:
                pairs = self.sim.extract_spikes(b["rec"], rows, b["rec_words"], pop.count)
                ticks_ = pairs[:, 0] + pop.window_start
                idx = pairs[:, 1]
            else:
                ticks_ = np.zeros(0, np.int64)
                idx = np.zeros(0, np.int64)
            if not self.lift_recording_budget and len(ticks_) > RECORDING_BUDGET:
                raise RuntimeError("event stream recording budget exceeded")
            if pop.spike_monitor:
                spike_ticks, indices = ticks_, idx
                counts = np.bincount(idx, minlength=pop.count).astype(np.int64)
            else:
                spike_ticks = indices = np.zeros(0, np.int64)
                counts = np.zeros(pop.count, np.int64)
            last_spikes = np.zeros(0, np.int64)
            if pop.has_spike_event and ran:
                slot = last_tick % pop.ring
                n_by_block = self.sim.read(b["spk_cnt"], np.uint32, pop.blocks, offset=slot * pop.blocks * 4)
                ids = self.sim.read(b["spk_ids"], np.uint32, pop.count, offset=slot * pop.count * 4)
                if self.launch_mode == "persistent":
                    ids &= RING_VALUE   # persistent launches stamp ring words with their tick
                last_spikes = np.concatenate(
                    [ids[k * plan.shape.block:k * plan.shape.block + int(n)] for k, n in enumerate(n_by_block)]
                ).astype(np.int64) if pop.blocks else last_spikes
            trace = {}
            if "mon_entries" in b:
                for name in pop.monitor_vars:
                    dtype = engine._var_dtype(pop, name)
                    trace[name] = self.sim.read(b[f"sample:{name}"], NUMPY[dtype],
                                                rows * len(pop.monitor_record)).reshape(rows, len(pop.monitor_record))
            else:
                for name in pop.monitor_vars:
                    trace[name] = np.zeros((rows, len(pop.monitor_record)), NUMPY[engine._var_dtype(pop, name)])
            refractory = None
            if pop.refractory is not None:
                if ran:
                    until = self.sim.read(b["until"], np.int32, pop.count)
                    available = until.astype(np.int64) <= last_tick
                else:
                    available = pop.refractory[2].astype(bool)
                refractory = {"lastspike": self.sim.read(b["lastspike"], np.float64, pop.count),
                              "not_refractory": available}
            streams = {"spike": {"ticks": ticks_, "indices": idx}} if pop.has_spike_event else {}
            for k, (event, _, _) in enumerate(pop.custom_events):
                # a custom event's stream: its bitmap rows over the recording window, like the spikes
                pairs = (self.sim.extract_spikes(b[f"evrec:{k}"], rows, b["rec_words"], pop.count) if rows
                         else np.zeros((0, 2), np.int64))
                if not self.lift_recording_budget and len(pairs) > RECORDING_BUDGET:
                    raise RuntimeError("event stream recording budget exceeded")
                streams[event] = {"ticks": pairs[:, 0] + pop.window_start, "indices": pairs[:, 1]}
            populations.append({"states": states, "trace": trace, "spike_ticks": spike_ticks, "indices": indices,
                                "counts": counts, "last_spikes": last_spikes, "refractory": refractory,
                                "event_streams": streams,
                                "event_monitors": self._event_monitors(pop)})
        delivered = self.sim.read(plan.delivered_buffer, np.uint64).reshape(-1, plan.total_blocks) \
            if plan.pathways else np.zeros((0, max(1, plan.total_blocks)), np.uint64)
        synapses = [{"states": {}, "events": 0, "edges": plan.synapse_edges[s]} for s in range(plan.synapse_count)]
        for post in plan.post_paths:
            synapses[post.synapse]["events"] += int(delivered[post.index].sum())
        for path in plan.pathways:
            entry = synapses[path.synapse]
            entry["events"] += int(delivered[path.index].sum())
            if path.state_owner is not None:   # its states are the owner pathway's records
                continue
            records = None
            if path.syn_states and path.edge_count:
                records = self.sim.read(path.buffers["syn"], np.uint8, path.edge_count * path.syn_stride) \
                    .view(engine.syn_record_dtype(path))
            for name, dtype, _ in path.syn_states:
                rows_values = np.ascontiguousarray(records[name]) if records is not None \
                    else np.zeros(0, NUMPY[dtype])
                if path.order is not None:
                    edge_values = np.empty_like(rows_values)
                    edge_values[path.order] = rows_values
                else:
                    edge_values = rows_values
                entry["states"][name] = edge_values
        return {"populations": populations, "synapses": synapses}

    def _event_monitors(self, pop) -> dict:
        """Each EventMonitor's (tick, neuron) events in the reference's order (tick, then neuron
        ascending: executor.rs:3053-3080 appends each tick's ascending fired list) and its
        values in their storage dtypes."""
        out = {}
        dtypes = {name: dtype for name, dtype, _ in pop.states}
        dtypes.update({name: dtype for name, (dtype, _) in pop.scalar_params.items()})
        dtypes.update({name: dtype for name, (dtype, _) in pop.vector_params.items()})
        for k, (name, variables, _, _) in enumerate(pop.event_monitors):
            count = int(self.sim.read(pop.buffers[f"emon_count:{k}"], np.uint32, 1)[0])
            if count > pop.event_monitor_capacity(k):
                raise RuntimeError("EventMonitor recording budget exceeded")
            width = 1 + len(variables)
            records = self.sim.read(pop.buffers[f"emon:{k}"], np.float64, count * width).reshape(count, width)
            key = records[:, 0].copy().view(np.uint64)
            ticks, neurons = (key >> np.uint64(32)).astype(np.int64), (key & np.uint64(0xFFFFFFFF)).astype(np.int64)
            order = np.lexsort((neurons, ticks))
            out[name] = {"ticks": ticks[order], "indices": neurons[order],
                         "values": {var: records[order, 1 + v].astype(NUMPY[dtypes[var]])
                                    for v, var in enumerate(variables)}}
        return out

    def close(self) -> None:
        if not self.closed:
            self.sim.close()
            self.closed = True

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
