#!/usr/bin/env python3
"""Throughput of the Brian2-Atlas simulation hot path on one MI355X.

Default workload (the largest single-GPU configuration
and the north-star target): scaled CUBA LIF, 1,000,000 neurons (80% excitatory),
fixed in-degree 1000 (800 excitatory + 200 inhibitory sources per target, 1e9
synapses, procedural topology built on the device), uniform delay of 1 tick,
dt = 0.1 ms, 1 s simulated (10,000 ticks), spike monitor on every neuron.
``--workload cuba1m_weighted`` is the same network with a float32 weight per synapse (the
storage BASELINE.json configs[2] names: int32 indices + float32 weights), drawn by a procedural
uniform initializer over [0.5, 1.5] x the constant weight, so delivery adds each event's own weight
in the reference's canonical order.
``--workload cuba4k`` runs configs[0] (CUBA, 4000 neurons, Bernoulli p = 0.02,
delay 0), ``--workload cobahh4k`` configs[1] (COBAHH, 4000 HH neurons),
``--workload plastic100k`` configs[4] (100k neurons, delays 1-20, STDP, 10 s
simulated: 100,000 ticks) and
``--workload rsnn`` configs[3] (recurrent LIF training: a step is one training
step, forward + BPTT + Adam, over a device-resident batch of 256 samples; the
value is samples/s, the roofline is fp32 MFMA FLOP/s of the dominant phase's
kernel).

A step is one full simulated second replayed from the initial snapshot (device
resident; the restore is device copies inside the timed region).  Reported:
synaptic events/s (the value), neuron updates/s and x realtime, the roofline of
the dominant kernel and a CPU baseline: the C restatement of the reference
executor (oracle/) timed on the host cores on a bounded sample of the same
workload.  ``--gpus N`` with N > 1 exits: this build runs one GPU.

Roofline: config 3 runs as one persistent cooperative launch of ``atlas_run``
per 10,000 ticks (the states stay in registers), otherwise as one launch of the
tick kernel per tick.  The average launch duration is the device time of the
timed steps, measured by HIP events recorded on the library's stream around
each run, divided by the launches.  Algorithmic bytes per tick: 28 B per neuron update
(v, ge, gi float32 read and write, 4 B refractory deadline; COBAHH: 6 states,
52 B) plus 4 B per delivered event (its target index; the weights are
per-pathway constants; 8 B with a weight per synapse: index and f32 weight), times the ticks a
launch runs.  ``traffic`` is the measured HBM bytes per launch
(rocprofv3 FETCH_SIZE and WRITE_SIZE, calibrated against a kernel of known
traffic), read from profiles/ when present.  With a delay-0 pathway (configs 1
and 2) each tick's launch delivers the previous tick and then updates its own, and
one more launch per run delivers the last tick; the roofline covers the tick.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "brian2-atlas_amd"))
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
BYTES_PER_EVENT = 4             # u32 target index per delivered event (weights are namespace constants)
BYTES_PER_WEIGHTED_EVENT = 8    # u32 target index + f32 weight per delivered event
BYTES_PER_PLASTIC_EVENT = 48    # row index + delay-ordered rank (8 B) + synapse state read (20 B) and written (20 B)
# One common scale of the CUBA weights (we, wi) for in-degree 1000: 0.0116 puts the
# mean rate at ~7.5 Hz, the middle of the configured 5-10 Hz band (CPU sweep with the
# oracle at 8000 neurons: 0.08 -> 2.1 Hz, 0.02 -> 5.1 Hz, 0.0116 -> 7.5 Hz, 0.008 -> 9.8 Hz).
CUBA_1M_WEIGHT_SCALE = 0.0116


def workload(args):
    """(document, description, config keys, bytes per neuron update, CPU-baseline document, sample text)."""
    from atlas_hip import models
    if args.workload in ("cuba1m", "cuba1m_weighted"):
        scale = args.weight_scale if args.weight_scale is not None else CUBA_1M_WEIGHT_SCALE
        weighted = args.workload == "cuba1m_weighted"
        doc = models.cuba_network(args.neurons, indegree=args.indegree, delay_ticks=1, steps=args.ticks,
                                  weight_scale=scale, dtype="f32", edge_weights=weighted)
        cpu = models.cuba_network(args.cpu_neurons, indegree=args.indegree, delay_ticks=1, steps=args.cpu_ticks,
                                  weight_scale=scale, dtype="f32", edge_weights=weighted)
        desc = (f"scaled CUBA LIF {args.neurons} neurons, fixed in-degree {args.indegree}, delay 1 tick, dt 0.1 ms, "
                f"{args.ticks * 1e-4:g} s simulated (BASELINE configs[2])"
                + (", f32 weight per synapse (uniform 0.5-1.5 x we, wi)" if weighted else ""))
        keys = {"neurons": args.neurons, "synapses": args.neurons * args.indegree, "weight_scale": scale}
        sample = (f"scaled CUBA, {args.cpu_neurons} neurons, fixed in-degree {args.indegree}, delay 1 tick, "
                  f"first {args.cpu_ticks} ticks")
        return doc, desc, keys, 28, cpu, sample
    if args.workload == "cuba4k":
        doc = models.cuba_network(4000, steps=args.ticks)
        desc = f"CUBA LIF 4000 neurons, Bernoulli p=0.02, delay 0, dt 0.1 ms, {args.ticks * 1e-4:g} s (BASELINE configs[0])"
        return doc, desc, {"neurons": 4000, "p": 0.02}, 28, doc, f"the same network, all {args.ticks} ticks"
    if args.workload == "cobahh4k":
        doc = models.cobahh_network(4000, steps=args.ticks)
        desc = (f"COBAHH 4000 HH neurons, exponential Euler, Bernoulli p=0.02, delay 0, dt 0.1 ms, "
                f"{args.ticks * 1e-4:g} s (BASELINE configs[1])")
        return doc, desc, {"neurons": 4000, "p": 0.02}, 52, doc, f"the same network, all {args.ticks} ticks"
    if args.workload == "plastic100k":
        doc = models.plastic_network(100_000, steps=args.ticks, packed=True)
        cpu_n = min(args.cpu_neurons, 10_000)
        cpu = models.plastic_network(cpu_n, steps=args.cpu_ticks, packed=False)
        desc = (f"plastic delayed CUBA LIF 100000 neurons, fixed in-degree 1000 (1e8 synapses), delays 1-20 ticks, "
                f"exc->exc STDP, dt 0.1 ms, {args.ticks * 1e-4:g} s (BASELINE configs[4])")
        return doc, desc, {"neurons": 100_000, "synapses": 100_000_000}, 28, cpu, \
            f"the same network at {cpu_n} neurons, first {args.cpu_ticks} ticks"
    raise SystemExit(f"unknown workload {args.workload!r}")


def log(*args):
    print(*args, file=sys.stderr, flush=True)


def cpu_neurons(args, keys) -> int:
    if args.workload in ("cuba1m", "cuba1m_weighted"):
        return args.cpu_neurons
    if args.workload == "plastic100k":
        return min(args.cpu_neurons, 10_000)
    return keys["neurons"]


def host_cpu() -> dict:
    """The host the CPU baseline ran on: CPU model (lscpu's "Model name", read from /proc/cpuinfo),
    logical CPUs the process may use (nproc) and those the machine has."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    return {"model": model, "nproc": usable, "logical_cpus": os.cpu_count(), "threads_used": 1}


def cpu_baseline(doc, sample: str, neurons: int) -> dict:
    """Time the oracle (single-threaded C restatement of b2-runner) on a bounded sample."""
    from oracle import oracle
    started = time.perf_counter()
    result = oracle.run(doc, lift_recording_budget=True)
    wall = time.perf_counter() - started
    sim = result.sim_seconds
    return {
        "value": result.synaptic_events / sim if sim > 0 else None,
        "unit": "events/s",
        "cores": 1,
        "kind": "port",
        "host": host_cpu(),
        "sample": (f"{sample}; {result.synaptic_events} events, {result.spike_count} spikes in "
                   f"{sim:.2f} s of simulation loop ({wall:.1f} s with model setup)"),
        "neuron_updates_per_s": neurons * result.ticks_run / sim if sim > 0 else None,
        "x_realtime": (result.ticks_run * 1e-4) / sim if sim > 0 else None,
    }


MFMA_FP32_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix peak


def rsnn_cpu_baseline(plan, x, labels, weights, seconds: float = 15.0) -> dict:
    """Time the float64 NumPy oracle of the trainer (forward, BPTT, Adam) on the host cores: whole
    training steps at the benchmark's shape, as many as fit in ``seconds``."""
    import numpy as np
    from oracle import rsnn_oracle
    try:
        from threadpoolctl import threadpool_info
        threads = max((int(i.get("num_threads", 1)) for i in threadpool_info() if i.get("user_api") == "blas"),
                      default=1)
    except ImportError:
        threads = None
    w = [a.astype(np.float64) for a in weights]
    moments = [(np.zeros_like(a), np.zeros_like(a)) for a in w]
    steps = 0
    started = time.perf_counter()
    while time.perf_counter() - started < seconds or steps == 0:
        fwd = rsnn_oracle.forward(plan, *w, x, labels)
        grads = rsnn_oracle.backward(plan, *w, x, fwd)
        steps += 1
        for k, key in enumerate(("w_in", "w_rec", "w_out")):
            w[k], moments[k] = rsnn_oracle.adam(w[k], moments[k], grads[key], steps, lr=plan["learning_rate"],
                                                beta1=plan["beta1"], beta2=plan["beta2"], epsilon=plan["epsilon"])
    wall = time.perf_counter() - started
    return {"value": round(steps * plan["batch"] / wall, 2), "unit": "samples/s", "cores": threads, "kind": "port",
            "sample": (f"{steps} float64 NumPy training steps (forward, BPTT, Adam) of the same batch of "
                       f"{plan['batch']} samples, {wall:.1f} s; cores = BLAS threads")}


def bench_rsnn(args) -> int:
    """Configuration 4: recurrent LIF training, samples/s over whole training steps."""
    import numpy as np
    from atlas_hip import rsnn
    plan = rsnn.recurrent_plan()
    rng = np.random.default_rng(args.seed)
    x, labels = rsnn.poisson_inputs(rng, plan["batch"], plan["time"], plan["inputs"], plan["classes"])
    weights = rsnn.initial_weights(plan, args.seed + 1)
    trainer = rsnn.NativeRecurrentTrainer(plan, weights=weights)
    trainer.set_batch(x, labels)
    for k in range(args.warmup):
        trainer.run(train=True)
        log(f"warmup {k}: {trainer.device_ms:.3f} ms device")
    device_ms = 0.0
    started = time.perf_counter()
    for k in range(args.steps):
        out = trainer.run(train=True)
        device_ms += trainer.device_ms
    wall = time.perf_counter() - started
    log(f"{args.steps} steps: {wall * 1e3 / args.steps:.3f} ms per step wall, "
        f"{device_ms / args.steps:.3f} ms device, last loss {out['loss']:.4f}")
    # per-phase device time (HIP events on the trainer's stream), averaged over profiled steps
    phases = {name: 0.0 for name in rsnn.PHASES}
    repeats = 20
    for _ in range(repeats):
        for name, ms in trainer.profile(train=True).items():
            phases[name] += ms / repeats
    trainer.close()
    B, T, H = plan["batch"], plan["time"], plan["hidden"]
    flops = rsnn.flops_per_sample(plan)
    step_flops = B * sum(flops.values())
    dominant = max(phases, key=phases.get)
    tick_phase = dominant in ("forward_ticks", "backward_ticks")
    if tick_phase:
        # hidden <= 256: one persistent launch per pass covers every tick; its recurrent products
        # are T - 1 (B x H) x (H x H) contractions (none on the first forward tick and the last
        # backward tick, which have no recurrent input)
        avg_launch_s = phases[dominant] * 1e-3
        per_launch = 2 * B * H * H * (T - 1)
        kernel = "forward_split" if dominant == "forward_ticks" else "backward_split"
    else:
        avg_launch_s = phases[dominant] * 1e-3
        per_launch = B * flops.get(dominant, 0)
        kernel = dominant
    achieved = per_launch / avg_launch_s / 1e12
    step_s = wall / args.steps
    line = {
        "metric": "training_samples_per_second", "value": round(B * args.steps / wall, 1), "unit": "samples/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_s * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic Poisson input (rates uniform 0-20 Hz per channel), random labels, random-init weights",
        "config": {"workload": ("recurrent LIF training, 700 -> 256 recurrent -> 20 leaky readout, T=100 x 1 ms, "
                                "batch 256, max-over-time cross-entropy, full BPTT, Adam lr 1e-3 "
                                "(BASELINE configs[3])"),
                   "batch": B, "time": T, "inputs": plan["inputs"], "hidden": H, "classes": plan["classes"]},
        "device_ms_per_step": round(device_ms / args.steps, 4),
        "phase_ms": {k: round(v, 4) for k, v in phases.items()},
        "algorithmic_gflop_per_step": round(step_flops / 1e9, 3),
        "step_mfma_frac": round(step_flops / (device_ms / args.steps * 1e-3) / 1e12 / MFMA_FP32_PEAK_TFLOPS, 4),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": MFMA_FP32_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / MFMA_FP32_PEAK_TFLOPS, 4), "traffic": None,
                     "kernel": kernel, "avg_launch_us": round(avg_launch_s * 1e6, 3),
                     "algorithmic_flops_per_launch": int(per_launch)},
        "cpu_baseline": None if args.no_cpu_baseline else rsnn_cpu_baseline(plan, x, labels, weights),
    }
    print(json.dumps(line), flush=True)
    return 0


def copy_probe() -> int:
    """Stream 1 GiB through an elementwise kernel five times: the reference reading of FETCH_SIZE /
    WRITE_SIZE (each dispatch reads exactly 1 GiB and writes 1 GiB; an elementwise kernel rather than
    copy_, which may run on the DMA engine where no kernel dispatch is counted)."""
    import torch
    nbytes = 1 << 30
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    started = time.perf_counter()
    for _ in range(5):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    seconds = (time.perf_counter() - started) / 5
    print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "dispatches": 5,
                      "GBps_read_plus_write": round(2 * nbytes / seconds / 1e9, 1)}), flush=True)
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=3)
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--workload", choices=["cuba1m", "cuba1m_weighted", "cuba4k", "cobahh4k", "plastic100k",
                                               "rsnn"],
                        default="cuba1m")
    parser.add_argument("--seed", type=int, default=0)
    parser.add_argument("--neurons", type=int, default=1_000_000)
    parser.add_argument("--indegree", type=int, default=1000)
    parser.add_argument("--ticks", type=int, default=None,
                        help="simulated ticks per step (default: the configuration's own, 10,000 or 100,000)")
    parser.add_argument("--weight-scale", type=float, default=None)
    parser.add_argument("--cpu-neurons", type=int, default=100_000)
    parser.add_argument("--cpu-ticks", type=int, default=3000)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-profile", action="store_true")
    parser.add_argument("--copy-probe", action="store_true",
                        help="only run a plain device copy of 1 GiB (counter calibration for rocprofv3 --pmc)")
    args = parser.parse_args()
    if args.ticks is None:
        args.ticks = 100_000 if args.workload == "plastic100k" else 10_000
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (no multi-GPU path); use --gpus 1", file=sys.stderr)
        return 2
    if args.copy_probe:
        return copy_probe()
    if args.workload == "rsnn":
        return bench_rsnn(args)

    from atlas_hip.executor import HipExecutor

    t0 = time.perf_counter()
    doc, desc, keys, bytes_per_neuron, cpu_doc, cpu_sample = workload(args)
    neurons = keys["neurons"]
    log(f"model built in {time.perf_counter() - t0:.1f} s")
    t0 = time.perf_counter()
    ex = HipExecutor(doc, device=0, lift_recording_budget=True, verify_envelope=False)
    log(f"executor ready in {time.perf_counter() - t0:.1f} s (setup {ex.setup_seconds:.1f} s, "
        f"compile {ex.compile_seconds:.2f} s)")
    for k in range(args.warmup):
        out = ex.run(collect=False)
        log(f"warmup {k}: {out['hip_runtime']['device_seconds']:.3f} s device")
    t0 = time.perf_counter()
    device_total = 0.0
    launches = 0
    for k in range(args.steps):
        out = ex.run(collect=False)
        device_total += out["hip_runtime"]["device_seconds"]
        launches += out["hip_runtime"]["launches"]
        log(f"step {k}: {out['hip_runtime']['device_seconds']:.3f} s device")
    wall = time.perf_counter() - t0
    if ex.plan.queues:
        log("delivery queues (records per arrival slot and block): " +
            ", ".join(f"pathway {k}: {q['cap']} of {q['limit']}" for k, q in ex.plan.queues.items()))
    result = ex.run(collect=True)
    spikes = int(sum(len(p["spike_ticks"]) for p in result["populations"]))
    events = int(sum(s["events"] for s in result["synapses"]))
    sim_seconds = args.ticks * ex.plan.dt
    step_seconds = wall / args.steps
    value = events / step_seconds
    log(f"spikes {spikes} ({spikes / neurons / sim_seconds:.2f} Hz), events {events}, "
        f"{step_seconds * 1e3:.1f} ms per simulated second")
    kernels = ex.plan.kernels
    persistent = ex.launch_mode == "persistent"
    plastic_events = int(result["synapses"][0]["events"]) if args.workload == "plastic100k" else 0
    # plastic events move their synapse state (w, Apre, Apost f32 + lastupdate f64, read and written)
    per_event = BYTES_PER_WEIGHTED_EVENT if args.workload == "cuba1m_weighted" else BYTES_PER_EVENT
    per_tick = bytes_per_neuron * neurons + (per_event * (events - plastic_events) +
                                             BYTES_PER_PLASTIC_EVENT * plastic_events) / args.ticks
    if persistent:
        # one cooperative launch runs up to PERSISTENT_TICKS ticks with the states in registers: its
        # algorithmic bytes are those of the ticks it runs, of which the states' share never
        # reaches HBM (the measured traffic shows what does)
        from atlas_hip import engine
        kernel = "atlas_run"
        ticks_per_launch = min(args.ticks, engine.PERSISTENT_TICKS)
        avg_s = device_total / launches
        per_launch = per_tick * ticks_per_launch
    else:
        kernel = kernels[0]
        ticks_per_launch = 1
        avg_s = device_total / (args.steps * args.ticks)   # one launch per tick (delay 0 adds one per run)
        per_launch = per_tick
    achieved = per_launch / avg_s / 1e9
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                "kernel": kernel, "avg_launch_us": round(avg_s * 1e6, 3), "launches": int(launches),
                "ticks_per_launch": ticks_per_launch, "us_per_tick": round(avg_s / ticks_per_launch * 1e6, 3),
                "algorithmic_bytes_per_launch": int(per_launch)}
    if args.workload == "cuba1m_weighted":
        traffic_name = "scaled_cuba_1M_weighted_persistent_traffic.json" if persistent else ""
    else:
        traffic_name = "scaled_cuba_1M_persistent_traffic.json" if persistent else "scaled_cuba_1M_traffic.json"
    traffic_file = ROOT / "profiles" / traffic_name
    if (traffic_name and traffic_file.exists() and args.workload in ("cuba1m", "cuba1m_weighted")
            and args.neurons == 1_000_000 and args.ticks == 10_000):
        measured = json.loads(traffic_file.read_text())
        # the counter runs cover fewer ticks per launch: scale the per-tick traffic to this launch
        roofline["traffic"] = int(measured["bytes_per_tick"] * ticks_per_launch)
    if not args.no_profile:
        # per-launch HIP event pairs (each pair adds its own recording overhead to the launch)
        ex.run(collect=False, profile=True)
        roofline["avg_launch_us_event_pairs"] = {
            name: round(ex.kernel_times[name][0] * 1e3 / ex.kernel_times[name][1], 3)
            for name in kernels if ex.kernel_times[name][1]}
    ex.close()
    line = {
        "metric": "synaptic_events_per_second", "value": round(value, 1), "unit": "events/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_seconds * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f64",
        "data": "synthetic",
        "config": {"workload": desc, **keys, "ticks": args.ticks, "storage": "f32 states, f64 registers"},
        "neuron_updates_per_s": round(neurons * args.ticks / step_seconds, 1),
        "x_realtime": round(sim_seconds / step_seconds, 3),
        "spikes_per_step": spikes, "events_per_step": events,
        "device_seconds_per_step": round(device_total / args.steps, 6),
        "roofline": roofline,
        "cpu_baseline": None if args.no_cpu_baseline else cpu_baseline(cpu_doc, cpu_sample, cpu_neurons(args, keys)),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
