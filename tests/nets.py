"""Small AtlasIR test networks shared by the CPU and GPU parity tests.

Each network is written with ``atlas_hip.models.NetworkBuilder`` and carries
the reference behaviour it re-expresses (file:line into the reference).
"""
from __future__ import annotations

import numpy as np

from atlas_hip import models, protocol
from atlas_hip.models import (DIMLESS, SECOND, VOLT, NetworkBuilder, add, div, ld, lit, mul, narrow, op, stmt,
                              sub, wide)

MASK = (1 << 64) - 1


def chronology_kat(dtype: str = "f32") -> dict:
    """Same-tick arrivals from three delay groups (test_metal_delays.py:49-93).

    Sources 0, 2, 1 fire at ticks 2, 1, 0 and reach target 0 through edges of
    delay 0, 1 and 2 with weights 1, -2**24, 2**24, so all three arrive at tick 2.
    Applied in the canonical order (emission tick ascending) the float32 sums are
    2**24, 0, 1; any other order loses the 1 to rounding or keeps 2**24.
    Expected final target ``v`` = [1, 0].
    """
    b = NetworkBuilder(dt=1e-4, steps=6, seed=1)
    onset = np.array([2, 0, 1], np.float64) * 1e-4
    # spike while t lies in [onset, onset + dt/2): exactly one tick per source
    threshold = op("and", op("ge", ld("t"), ld("onset")),
                   op("lt", ld("t"), add(ld("onset"), mul(lit(0.5), ld("dt")))))
    src = b.population("source", 3, states={"v": ("f64", DIMLESS, np.zeros(3))},
                       parameters={"onset": ("f64", SECOND, onset)}, threshold=threshold)
    tgt = b.population("target", 2, states={"v": (dtype, DIMLESS, np.zeros(2))}, spike_monitor=False)
    w = wide if dtype == "f32" else (lambda e: e)
    nr = narrow if dtype == "f32" else (lambda e: e)
    b.projection("synapses", src, tgt, on_pre=[stmt("v", dtype, nr(add(w(ld("v")), w(ld("w")))))],
                 post_aliases={"v": "v"}, parameters={"w": ("f32", DIMLESS, np.array([1.0, -2.0**24, 2.0**24]))},
                 explicit=(np.array([0, 2, 1]), np.array([0, 0, 0])), delay_ticks=np.array([0, 1, 2]))
    return b.document()


def readme_lif(dt: float = 1e-4, steps: int = 1000) -> dict:
    """The README first simulation (README.md:113-124): one neuron,
    dv/dt = (1.5 - v)/(10 ms), threshold v > 1, reset v = 0, Euler, 100 ms -> 9 spikes."""
    b = NetworkBuilder(dt=dt, steps=steps, seed=1)
    update = ([], [stmt("_v", "f64", add(ld("v"), div(mul(ld("dt"), sub(lit(1.5), ld("v"))), ld("tau")))),
                   stmt("v", "f64", ld("_v"))])
    b.population("neurongroup", 1, states={"v": ("f64", DIMLESS, np.zeros(1))},
                 parameters={"tau": ("f64", SECOND, 10e-3)}, update=update,
                 threshold=op("gt", ld("v"), lit(1.0)), reset=[stmt("v", "f64", lit(0.0))])
    return b.document()


# ------------------------------------------------- recurrent CUBA comparison workload
RECURRENT = dict(dt=1e-4, tau=20e-3, syn_tau=5e-3, ref_ticks=20, delay_ticks=20, weights=(0.05, -0.2))


def recurrent_arrays(neurons: int, degree: int):
    """Inputs of the reference's recurrent comparison workload (gpu_recurrent.py:33-52).

    Initial v = (37 i mod 1024)/1024 and drive = 1.15 + 0.02 (i mod 7), both
    float32; per target and projection kind, sources are drawn by a splitmix64
    stream seeded with 1729 + 2 target + kind, rejecting repeats, until the
    projection's in-degree is reached (80/20 split of ``degree``).
    """
    ne = int(0.8 * neurons)
    ki = max(1, degree // 5)
    ke = degree - ki
    index = np.arange(neurons)
    initial = ((index * 37 % 1024) / 1024).astype(np.float32)
    drive = (1.15 + (index % 7) * 0.02).astype(np.float32)
    projections = []
    for kind, (start, size, count, weight) in enumerate(((0, ne, ke, 0.05), (ne, neurons - ne, ki, -0.2))):
        sources, targets = [], []
        for target in range(neurons):
            state = 1729 + 2 * target + kind
            chosen: set[int] = set()
            while len(chosen) < count:
                state = (state + 0x9E3779B97F4A7C15) & MASK
                z = ((state ^ (state >> 30)) * 0xBF58476D1CE4E5B9) & MASK
                z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
                z ^= z >> 31
                source = start + z % size
                if source not in chosen:
                    chosen.add(source)
                    sources.append(source)
                    targets.append(target)
        projections.append((np.asarray(sources, np.int64), np.asarray(targets, np.int64), np.float32(weight)))
    return initial, drive, projections


def recurrent_network(neurons: int = 400, degree: int = 50, steps: int = 2000) -> dict:
    """The recurrent comparison workload as AtlasIR (gpu_recurrent.py:78-93):
    Euler ``dv/dt = (drive - v + I_syn)/(20 ms)`` (unless refractory),
    ``dI_syn/dt = -I_syn/(5 ms)``, v > 1 -> v = 0, refractory 20 ticks, on_pre
    ``I_syn += w`` with delay 20 ticks, float32 states."""
    c = RECURRENT
    initial, drive, projections = recurrent_arrays(neurons, degree)
    b = NetworkBuilder(dt=c["dt"], steps=steps, seed=1729)
    v_new = add(wide(ld("v")), div(mul(ld("dt"), add(sub(wide(ld("drive")), wide(ld("v"))), wide(ld("I_syn")))),
                                   ld("tau")))
    i_new = sub(wide(ld("I_syn")), div(mul(ld("dt"), wide(ld("I_syn"))), ld("syn_tau")))
    update = ([], [stmt("_v", "f32", narrow(v_new), DIMLESS, "not_refractory"),
                   stmt("_I_syn", "f32", narrow(i_new)),
                   stmt("v", "f32", ld("_v"), DIMLESS, "not_refractory"),
                   stmt("I_syn", "f32", ld("_I_syn"))])
    pop = b.population("population", neurons,
                       states={"v": ("f32", DIMLESS, initial), "I_syn": ("f32", DIMLESS, np.zeros(neurons))},
                       parameters={"drive": ("f32", DIMLESS, drive), "tau": ("f64", SECOND, c["tau"]),
                                   "syn_tau": ("f64", SECOND, c["syn_tau"])},
                       update=update, threshold=op("gt", wide(ld("v")), lit(1.0)),
                       reset=[stmt("v", "f32", narrow(lit(0.0)))],
                       refractory=c["ref_ticks"] * c["dt"])
    for label, (sources, targets, weight) in zip(("exc", "inh"), projections):
        b.projection(label, pop, pop, on_pre=[stmt("I_syn", "f32", narrow(add(wide(ld("I_syn")), wide(ld("w")))))],
                     post_aliases={"I_syn": "I_syn"},
                     parameters={"w": ("f32", DIMLESS, np.full(sources.size, weight, np.float32))},
                     explicit=(sources, targets), delay_ticks=c["delay_ticks"])
    return b.document()


def recurrent_reference(neurons: int, degree: int, steps: int) -> dict:
    """Independent f64 Euler/event evaluation of the recurrent workload
    (the method of gpu_recurrent.py:54-74: dense per-tick arrays, integer
    refractory deadlines, delay buckets keyed by arrival tick); initial arrays
    keep their float32 values.  Accumulation uses a dense (source, target)
    weight matrix, a different route from the executor's per-event programs."""
    c = RECURRENT
    initial, drive, projections = recurrent_arrays(neurons, degree)
    v = initial.astype(np.float64)
    drive = drive.astype(np.float64)
    weights = np.zeros((neurons, neurons))
    for sources, targets, weight in projections:
        np.add.at(weights, (sources, targets), float(weight))
    current = np.zeros(neurons)
    until = np.zeros(neurons, np.int64)
    pending: dict[int, np.ndarray] = {}
    ticks, indices = [], []
    dt_ms, tau_ms, syn_ms = c["dt"] * 1e3, c["tau"] * 1e3, c["syn_tau"] * 1e3
    for tick in range(steps):
        free = tick >= until
        v[free] += dt_ms * (drive[free] - v[free] + current[free]) / tau_ms
        current -= dt_ms * current / syn_ms
        fired = np.flatnonzero(free & (v > 1))
        ticks.extend([tick] * fired.size)
        indices.extend(fired.tolist())
        pending[tick + c["delay_ticks"]] = fired
        arriving = pending.pop(tick, None)
        if arriving is not None and arriving.size:
            current += weights[arriving].sum(axis=0)
        v[fired] = 0.0
        until[fired] = tick + c["ref_ticks"]
    return dict(v=v, I_syn=current, ticks=np.asarray(ticks, np.int64), indices=np.asarray(indices, np.int64))


def weighted_burst(n: int = 3000, indegree: int = 200, steps: int = 30, seed: int = 5) -> dict:
    """Voltage-jump LIF with distinct float32 weights per edge (so deliveries are ordered,
    not counted) and every neuron starting above threshold: tick 1 delivers all n * indegree
    events at once, many times the LDS staging capacity of a block."""
    rng = np.random.default_rng(seed)
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    taum, El, Vt, Vr = 20e-3, -55e-3, -50e-3, -60e-3
    scalar = [stmt("_lio_1", "f64", models.un("exp", div(models.neg(ld("dt")), ld("taum"))))]
    vector = [stmt("_v", "f32", narrow(add(ld("El"), mul(sub(wide(ld("v")), ld("El")), ld("_lio_1")))), VOLT,
                   "not_refractory"),
              stmt("v", "f32", ld("_v"), VOLT, "not_refractory")]
    pop = b.population("neurongroup", n, states={"v": ("f32", VOLT, np.full(n, -49.5e-3))},
                       parameters={"taum": ("f64", SECOND, taum), "El": ("f64", VOLT, El),
                                   "Vt": ("f64", VOLT, Vt), "Vr": ("f64", VOLT, Vr)},
                       update=(scalar, vector), threshold=op("gt", wide(ld("v")), ld("Vt")),
                       reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=1e-3)
    sources = np.concatenate([rng.choice(n, indegree, replace=False) for _ in range(n)])
    targets = np.repeat(np.arange(n), indegree)
    weights = rng.uniform(-0.2e-3, 0.25e-3, sources.size).astype(np.float32)
    b.projection("synapses", pop, pop, on_pre=[stmt("v", "f32", narrow(add(wide(ld("v")), wide(ld("w")))), VOLT)],
                 post_aliases={"v": "v"}, parameters={"w": ("f32", VOLT, weights)},
                 explicit=(sources, targets), delay_ticks=1)
    return b.document()


# ------------------------------------------------- HH ionic comparison workload
HH_ACCEPT = dict(rtol=3e-4, atol=dict(v=5e-6, m=2e-5, n=2e-5, h=2e-5, ge=1e-12, gi=1e-12))


def hh_arrays(neurons: int) -> dict:
    """Deterministic float32 inputs of the reference's HH workload (gpu_hh.py:52-56)."""
    i = np.arange(neurons)
    return dict(v=np.asarray(-0.065 + (i % 11 - 5) * 0.0005, np.float32), m=np.zeros(neurons, np.float32),
                n=np.zeros(neurons, np.float32), h=np.zeros(neurons, np.float32),
                ge=np.asarray((i % 7 + 1) * 8e-9, np.float32), gi=np.asarray((i % 5) * 20e-9, np.float32),
                I_ext=np.asarray((0.2 + (i % 9) * 0.05) * 1e-9, np.float32))


def hh_ionic_network(neurons: int = 64, steps: int = 2000, dtype: str = "f32") -> dict:
    """HH ionic dynamics with a constant injected current and no synapses (gpu_hh.py:21-49):
    the COBAHH rates and exponential-Euler update, threshold v > -20 mV, refractory 30 ticks
    suppressing spikes only, float32 states."""
    from atlas_hip.models import SIEMENS, _hh_parameters, hh_update
    a = hh_arrays(neurons)
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=1)
    params = _hh_parameters()
    # the workload's constants (gpu_hh.py:13-24): Cm 200 pF, gl 10 nS, gNa 20 uS, gK 6 uS
    params.update(Cm=("f64", models.FARAD, 2e-10), gl=("f64", SIEMENS, 1e-8), g_na=("f64", SIEMENS, 2e-5),
                  g_kd=("f64", SIEMENS, 6e-6), I_ext=("f32", models.AMP, a["I_ext"]))
    w = wide if dtype == "f32" else (lambda e: e)
    b.population("population", neurons,
                 states={k: (dtype, VOLT if k == "v" else SIEMENS if k in ("ge", "gi") else DIMLESS, a[k])
                         for k in ("v", "m", "n", "h", "ge", "gi")},
                 parameters=params, update=hh_update(dtype, external_current=True),
                 threshold=op("gt", w(ld("v")), lit(-0.020)), refractory=30e-4, frozen=())
    return b.document()


def hh_reference(neurons: int, steps: int) -> dict:
    """Independent f64 evaluation of the HH workload (the method of gpu_hh.py:59-89): the
    equilibrium/expm1 form of exponential Euler, initial arrays at their float32 values."""
    a = {k: v.astype(np.float64) for k, v in hh_arrays(neurons).items()}
    cm, gl, gna, gk, el, ena, ek, vt, ee, ei, dt = 2e-10, 1e-8, 2e-5, 6e-6, -0.060, 0.050, -0.090, -0.063, 0.0, -0.080, 1e-4

    def exprel(x):
        return np.divide(np.expm1(x), x, out=np.ones_like(x), where=x != 0)

    until = np.zeros(neurons, np.int64)
    ticks, indices = [], []
    for tick in range(steps):
        v, m, n, h, ge, gi = (a[k] for k in ("v", "m", "n", "h", "ge", "gi"))
        g_na, g_k = gna * m ** 3 * h, gk * n ** 4
        g = gl + ge + gi + g_na + g_k
        eq = (gl * el + ge * ee + gi * ei + g_na * ena + g_k * ek + a["I_ext"]) / g
        v_next = v + (eq - v) * (-np.expm1(-dt * g / cm))
        rates = {"m": (1280 / exprel((0.013 - v + vt) / 0.004), 1400 / exprel((v - vt - 0.040) / 0.005)),
                 "h": (128 * np.exp((0.017 - v + vt) / 0.018), 4000 / (1 + np.exp((0.040 - v + vt) / 0.005))),
                 "n": (160 / exprel((0.015 - v + vt) / 0.005), 500 * np.exp((0.010 - v + vt) / 0.040))}
        for name, (alpha, beta) in rates.items():
            old = a[name]
            a[name] = old + (alpha / (alpha + beta) - old) * (-np.expm1(-dt * (alpha + beta)))
        a.update(v=v_next, ge=ge * np.exp(-dt / 0.005), gi=gi * np.exp(-dt / 0.010))
        fired = np.flatnonzero((tick >= until) & (v_next > -0.020))
        ticks.extend([tick] * fired.size)
        indices.extend(fired.tolist())
        until[fired] = tick + 30
    return {**{k: a[k] for k in ("v", "m", "n", "h", "ge", "gi")}, "ticks": np.asarray(ticks, np.int64),
            "indices": np.asarray(indices, np.int64)}


# ------------------------------------------------- delayed recurrent STDP workload
STDP = dict(dt=1.0 / 1024, drive=0.125, delay_span=4, post_delay=2, taupre_ticks=16, taupost_ticks=32,
            dapre=0.0078125, dapost=-0.00390625, wmax=0.5, w0=0.25)


def stdp_ring(neurons: int, degree: int):
    """Ring topology of the reference's STDP workload (gpu_stdp_compare.py:37-60): source s
    connects to s+1 .. s+degree (mod N) in that creation order; edge e has delay e mod 4."""
    sources = np.repeat(np.arange(neurons, dtype=np.int64), degree)
    targets = (sources + np.tile(np.arange(degree), neurons) + 1) % neurons
    return sources, targets, np.arange(sources.size, dtype=np.int64) % STDP["delay_span"]


def stdp_network(neurons: int = 64, degree: int = 8, steps: int = 400) -> dict:
    """The reference's delayed recurrent STDP workload as AtlasIR (gpu_stdp_compare.py:63-87),
    float64 states:
      neuron: v += drive then v += -v/32 each tick, v > 1 -> v = 0, v0 = (i mod 16)/16;
      on_pre (delay e mod 4): decay Apre (tau 16 ticks) and Apost (tau 32 ticks) since lastupdate,
        v_post += w/16, Apre += 1/128, w = clip(w + Apost, 0, 0.5), lastupdate = t;
      on_post (delay 2): decay both, Apost -= 1/256, w = clip(w + Apre, 0, 0.5), lastupdate = t.
    """
    c = STDP
    dt = c["dt"]
    b = NetworkBuilder(dt=dt, steps=steps, seed=1)
    update = ([], [stmt("_v1", "f64", add(ld("v"), lit(c["drive"]))),
                   stmt("v", "f64", add(ld("_v1"), mul(lit(-1.0 / 32), ld("_v1"))))])
    pop = b.population("neurongroup", neurons, states={"v": ("f64", DIMLESS, (np.arange(neurons) % 16) / 16)},
                       update=update, threshold=op("gt", ld("v"), lit(1.0)), reset=[stmt("v", "f64", lit(0.0))])
    sources, targets, delays = stdp_ring(neurons, degree)
    elapsed = sub(ld("t"), ld("lastupdate"))
    decay = [stmt("Apre", "f64", mul(ld("Apre"), models.un("exp", div(models.neg(elapsed), lit(c["taupre_ticks"] * dt))))),
             stmt("Apost", "f64", mul(ld("Apost"), models.un("exp", div(models.neg(elapsed), lit(c["taupost_ticks"] * dt)))))]
    clip = lambda x: {"op": "clip", "value": x, "min": lit(0.0), "max": lit(c["wmax"])}  # noqa: E731
    on_pre = decay + [stmt("v", "f64", add(ld("v"), div(ld("w"), lit(16.0)))),
                      stmt("Apre", "f64", add(ld("Apre"), lit(c["dapre"]))),
                      stmt("w", "f64", clip(add(ld("w"), ld("Apost")))),
                      stmt("lastupdate", "f64", ld("t"), SECOND)]
    on_post = decay + [stmt("Apost", "f64", add(ld("Apost"), lit(c["dapost"]))),
                       stmt("w", "f64", clip(add(ld("w"), ld("Apre")))),
                       stmt("lastupdate", "f64", ld("t"), SECOND)]
    e = sources.size
    b.projection("synapses", pop, pop, on_pre=on_pre, on_post=on_post, post_aliases={"v": "v"},
                 states={"w": ("f64", DIMLESS, np.full(e, c["w0"])), "Apre": ("f64", DIMLESS, np.zeros(e)),
                         "Apost": ("f64", DIMLESS, np.zeros(e)), "lastupdate": ("f64", SECOND, np.zeros(e))},
                 explicit=(sources, targets), delay_ticks=delays, post_delay_ticks=c["post_delay"])
    return b.document()


def stdp_reference(neurons: int, degree: int, steps: int) -> dict:
    """Independent ordered event recurrence of the STDP workload (the method of
    gpu_stdp_compare.py:90-117): per tick drive and leak, threshold, on_pre events in
    (emission tick, source, edge) order, then on_post events, then the reset."""
    c = STDP
    dt = c["dt"]
    source, target, delay = stdp_ring(neurons, degree)
    edges = source.size
    v = (np.arange(neurons) % 16 / 16).astype(np.float64)
    w = np.full(edges, c["w0"])
    ap = np.zeros(edges)
    ao = np.zeros(edges)
    last = np.zeros(edges)
    history = np.zeros((steps, neurons), bool)
    ticks, indices = [], []
    order = np.lexsort((np.arange(edges), source, -delay))
    for tick in range(steps):
        v += c["drive"]
        v += (-1 / 32) * v
        fired = v > 1
        history[tick] = fired
        spiking = np.flatnonzero(fired)
        ticks.extend([tick] * spiking.size)
        indices.extend(spiking.tolist())
        pre = order[(tick >= delay[order]) & history[np.maximum(tick - delay[order], 0), source[order]]]
        post = np.flatnonzero(history[tick - c["post_delay"], target]) if tick >= c["post_delay"] \
            else np.empty(0, np.int64)
        for events, is_pre in ((pre, True), (post, False)):
            elapsed = tick * dt - last[events]
            ap[events] *= np.exp(-elapsed / (c["taupre_ticks"] * dt))
            ao[events] *= np.exp(-elapsed / (c["taupost_ticks"] * dt))
            if is_pre:
                for k in events:                      # sequential: same-target order matters
                    v[target[k]] += w[k] / 16
                ap[events] += c["dapre"]
                w[events] = np.clip(w[events] + ao[events], 0, c["wmax"])
            else:
                ao[events] += c["dapost"]
                w[events] = np.clip(w[events] + ap[events], 0, c["wmax"])
            last[events] = tick * dt
        v[fired] = 0
    return dict(v=v, w=w, Apre=ap, Apost=ao, lastupdate=last, ticks=np.asarray(ticks, np.int64),
                indices=np.asarray(indices, np.int64))


def weighted_cuba(n=1000, steps=300, seed=3):
    """CUBA with a per-edge excitatory weight (an ordered on_pre: it reads per-edge data)."""
    doc = protocol.load(models.cuba_network(n, steps=steps, delay_ticks=1), verify_envelope=False)
    doc.pop("protocol", None)
    sdef, sin = doc["definition"]["synapses"][0], doc["instance"]["synapses"][0]
    we = next(p for p in sdef["parameters"] if p["name"] == "we")
    we["index_domain"] = "synapse"
    base = float(np.frombuffer(bytes.fromhex(sin["parameters"]["we"][0]), ">f8")[0])
    scale = np.random.default_rng(seed).uniform(0.5, 1.5, len(sin["source"]))
    sin["parameters"]["we"] = models.hex_array(base * scale, "f64")
    return protocol.seal(doc)


def noisy_lif(n: int = 2000, steps: int = 500, sigma: float = 3e-3, seed: int = 11) -> dict:
    """LIF with white-noise input, Euler-Maruyama as Brian2 lowers ``sigma * xi * tau**-0.5``:
    v <- v + dt (El - v) / tau + sigma sqrt(dt / tau) randn(); threshold v > Vt, reset Vr,
    refractory 2 ms; f32 storage."""
    builder = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    rng = np.random.default_rng(seed)
    vector = [stmt("v", "f32", narrow(add(add(wide(ld("v")), div(mul(ld("dt"), models.sub(ld("El"), wide(ld("v")))), ld("tau"))),
                                          mul(mul(ld("sigma"), models.un("sqrt", div(ld("dt"), ld("tau")))),
                                              {"op": "randn", "stream": 1}))), VOLT)]
    builder.population(
        "noisy", n, states={"v": ("f32", VOLT, rng.uniform(-60e-3, -50e-3, n))},
        parameters={"tau": ("f64", SECOND, 10e-3), "El": ("f64", VOLT, -52e-3), "Vt": ("f64", VOLT, -50e-3),
                    "Vr": ("f64", VOLT, -60e-3), "sigma": ("f64", VOLT, sigma)},
        update=([], vector), threshold=op("gt", wide(ld("v")), ld("Vt")),
        reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=2e-3)
    return builder.document()


def nonfinite_network(kind: str, steps: int, n: int = 1000, bad: int = 123) -> dict:
    """A population whose neuron `bad` makes an intermediate value non-finite after a few ticks,
    while every other neuron stays finite.  The f64 intermediate is the operand of an f32
    rounding ("overflow": v <- f32(v * 1e3), v0 = 1e30, infinite in f32 at tick 2), of a clip
    whose result stays finite ("clip": x <- clip(v * 1e300, 0, 1) with v <- 10 v), of a divisor
    whose quotient is zero ("divisor": x <- 1 / (v * 1e300)) or of a negation under exp
    ("exp": x <- exp(-(v * 1e300)), zero).  "events": ten spike sources firing every tick each
    add 1e37 to x of neuron `bad` (x <- f32(x + w), counted events of delay 1): x passes the f32
    range at the 35th event, the fifth of the fourth tick's ten.  Both engines must fail at the
    same tick count."""
    builder = NetworkBuilder(dt=1e-4, steps=steps, seed=5)
    rng = np.random.default_rng(17)
    v0 = rng.uniform(0.5, 1.0, n)
    v0[bad] = 1e30 if kind == "overflow" else 0.75 if kind == "events" else 1e5
    grow = lit(1e3 if kind == "overflow" else 10.0)
    vector = [stmt("v", "f32", narrow(mul(wide(ld("v")), grow)), DIMLESS)]
    big = mul(wide(ld("v")), lit(1e300))
    if kind == "clip":
        vector.append(stmt("x", "f32", narrow({"op": "clip", "value": big, "min": lit(0.0), "max": lit(1.0)}),
                           DIMLESS))
    elif kind == "divisor":
        vector.append(stmt("x", "f32", narrow(div(lit(1.0), big)), DIMLESS))
    elif kind == "exp":
        vector.append(stmt("x", "f32", narrow(models.un("exp", models.neg(big))), DIMLESS))
    target = builder.population(
        "nonfinite", n, states={"v": ("f32", DIMLESS, v0), "x": ("f32", DIMLESS, np.zeros(n))},
        update=([], vector), threshold=op("gt", wide(ld("v")), lit(3.0e38)))
    if kind == "events":
        drive = builder.spike_generator("drive", 10, np.repeat(np.arange(steps), 10), np.tile(np.arange(10), steps))
        builder.projection("syn", drive, target, on_pre=[stmt("x", "f32", narrow(add(wide(ld("x")), ld("w"))))],
                           explicit=(np.arange(10), np.full(10, bad)), post_aliases={"x": "x"},
                           parameters={"w": ("f64", DIMLESS, 1e37)}, delay_ticks=1)
    return builder.document()


def procedural_cuba(n: int = 100_000, *, indegree: int = 100, steps: int = 300, seed: int = 1729,
                    weight_scale: float = 0.3) -> dict:
    """CUBA with procedural projections drawn entirely by the engine: excitatory sources by fixed
    in-degree with per-edge weights Uniform(0.5, 1.5) * we, inhibitory ones by fixed total
    (n * indegree / 4 edges, with replacement) with ClippedNormal(wi, |wi| / 4, max 0) weights, and
    both pathways' delays from Uniform(0.05 ms, 2 ms) initializers (1..20 ticks after
    floor(delay/dt + 0.5)).  Per-edge weights make the deliveries ordered."""
    c = models.CUBA
    rng = np.random.default_rng(seed)
    n_exc = int(round(n * 0.8))
    builder = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    zeros = np.zeros(n)
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    P = builder.population(
        "neurongroup", n,
        states={"v": ("f32", VOLT, c["Vr"] + rng.random(n) * (c["Vt"] - c["Vr"])), "ge": ("f32", VOLT, zeros),
                "gi": ("f32", VOLT, zeros)},
        parameters={"taum": scalar(c["taum"], SECOND), "taue": scalar(c["taue"], SECOND),
                    "taui": scalar(c["taui"], SECOND), "El": scalar(c["El"], VOLT),
                    "Vt": scalar(c["Vt"], VOLT), "Vr": scalar(c["Vr"], VOLT)},
        update=models.cuba_update("f32"), threshold=op("gt", wide(ld("v")), ld("Vt")),
        reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=c["refractory"])
    we, wi = c["we"] * weight_scale, c["wi"] * weight_scale
    delay = models.initializer_uniform(0.05e-3, 2e-3)
    builder.projection("exc", P, P, on_pre=[stmt("ge", "f32", narrow(add(wide(ld("ge")), ld("w"))), VOLT)],
                       source_range=(0, n_exc), post_aliases={"ge": "ge"}, parameters={"w": ("f64", VOLT, None)},
                       fixed_indegree=int(round(indegree * 0.8)),
                       initializers={"w": models.initializer_uniform(0.5 * we, 1.5 * we)}, delay_initializer=delay)
    builder.projection("inh", P, P, on_pre=[stmt("gi", "f32", narrow(add(wide(ld("gi")), ld("w"))), VOLT)],
                       source_range=(n_exc, n), post_aliases={"gi": "gi"}, parameters={"w": ("f64", VOLT, None)},
                       fixed_total=n * indegree // 4,
                       initializers={"w": models.initializer_clipped_normal(wi, abs(wi) / 4, None, 0.0)},
                       delay_initializer=delay)
    return builder.document()


# --------------------------------------------- procedural topology with initializers
INIT_SEED = 0x12345678
INIT_DT = 1.0 / 1024


def initialization_network(kind: str, distribution: str) -> dict:
    """The model of test_gpu_initialization.py:63-76: 8 spike sources firing every tick
    (SpikeGeneratorGroup with period dt), 7 targets, a Synapses onto targets 1..5 with
    ``v_post += w``; the topology is ``connect_fixed_total(257)`` or
    ``connect_fixed_indegree(3)`` with seed 0x12345678, w drawn by
    Uniform(0.0625, 0.25) or ClippedNormal(0.125, 0.03, 0.0625, 0.25) on stream 2,
    the on_pre delays by Uniform(0, 3 dt) or ClippedNormal(1.5 dt, 0.5 dt, 0, 3 dt) on
    stream 4, dt = 1/1024 s, 8 ticks, v of every target recorded."""
    b = NetworkBuilder(dt=INIT_DT, steps=8, seed=1)
    ticks = [t for t in range(8) for _ in range(8)]
    indices = [i for _ in range(8) for i in range(8)]
    src = b.spike_generator("source", 8, ticks, indices)
    tgt = b.population("target", 7, states={"v": ("f32", DIMLESS, np.zeros(7))}, spike_monitor=False,
                       state_monitor=(["v"], list(range(7))))
    if distribution == "uniform":
        weight = models.initializer_uniform(0.0625, 0.25)
        delay = models.initializer_uniform(0.0, 3 * INIT_DT)
    else:
        weight = models.initializer_clipped_normal(0.125, 0.03, 0.0625, 0.25)
        delay = models.initializer_clipped_normal(1.5 * INIT_DT, 0.5 * INIT_DT, 0.0, 3 * INIT_DT)
    b.projection("synapses", src, tgt, on_pre=[stmt("v", "f32", narrow(add(wide(ld("v")), wide(ld("w")))))],
                 target_range=(1, 6), post_aliases={"v": "v"}, parameters={"w": ("f32", DIMLESS, None)},
                 fixed_total=257 if kind == "total" else None, fixed_indegree=None if kind == "total" else 3,
                 topology_seed=INIT_SEED, initializers={"w": weight}, delay_initializer=delay)
    return b.document()


def initialization_draw(stream: int, index: int, attempt: int = 0) -> int:
    """``draw`` of test_gpu_initialization.py:29-36 (the topology splitmix64 with the golden-gamma pre-add)."""
    x = (INIT_SEED ^ ((stream * 0xD2B74407B1CE6E93) & MASK) ^ ((index * 0x9E3779B97F4A7C15) & MASK)
         ^ ((attempt * 0xCA5A826395121157) & MASK))
    x = (x + 0x9E3779B97F4A7C15) & MASK
    x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & MASK
    x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & MASK
    return x ^ (x >> 31)


def initialization_uniform(stream: int, index: int, attempt: int = 0) -> float:
    """``uniform`` of test_gpu_initialization.py:39: the open-interval 53-bit uniform."""
    return ((initialization_draw(stream, index, attempt) >> 11) + .5) / 2**53


def initialization_normal(stream: int, index: int, mean: float, std: float, low: float, high: float) -> float:
    """``normal`` of test_gpu_initialization.py:42-47: Box-Muller on streams (stream, stream + 1),
    attempts 2a and 2a + 1, rejected until inside [low, high]."""
    import math
    for attempt in range(1000):
        z = math.sqrt(-2 * math.log(initialization_uniform(stream, index, 2 * attempt))) * \
            math.cos(math.tau * initialization_uniform(stream + 1, index, 2 * attempt + 1))
        value = mean + std * z
        if low <= value <= high:
            return value
    raise AssertionError("unexpected rejection exhaustion")


def initialization_endpoints(kind: str) -> np.ndarray:
    """``endpoints`` of test_gpu_initialization.py:50-60: (source, target) pairs of the
    8 -> 5 topology, stably sorted by source."""
    pairs = []
    if kind == "total":
        pairs = [((initialization_draw(0, e) * 8) >> 64, (initialization_draw(1, e) * 5) >> 64) for e in range(257)]
    else:
        for target in range(5):
            selected: set[int] = set()
            for candidate in range(5, 8):
                value = (initialization_draw(0, target * 8 + candidate) * (candidate + 1)) >> 64
                source = candidate if value in selected else value
                selected.add(source)
                pairs.append((source, target))
    return np.asarray(sorted(pairs, key=lambda pair: pair[0]), dtype=np.uint32)


def initialization_expected(kind: str, distribution: str, f32_weights: bool = False) -> dict:
    """The expected run of test_gpu_initialization.py:79-101: per-edge weights and delay
    ticks floor(delay/dt + 0.5), then 8 ticks of deliveries in the order (delay descending,
    source, edge), the trace taken before each tick's deliveries.  With ``f32_weights`` each
    weight is rounded to float32 before the float32 add, as the reference's float32 GPU
    test writes it; otherwise the float32 target adds the f64 weight and rounds once, as the
    CPU engine's f64 registers do (executor.rs:457-466, 6214-6244)."""
    edges = initialization_endpoints(kind)
    count = len(edges)
    if distribution == "uniform":
        weights = np.array([.0625 + .1875 * initialization_uniform(2, e) for e in range(count)])
        delays = np.array([3 * initialization_uniform(4, e) for e in range(count)])
    else:
        weights = np.array([initialization_normal(2, e, .125, .03, .0625, .25) for e in range(count)])
        delays = np.array([initialization_normal(4, e, 1.5, .5, 0, 3) for e in range(count)])
    ticks = np.floor(delays + .5).astype(int)
    v = np.zeros(7, np.float32)
    trace, events = [], 0
    order = sorted(range(count), key=lambda e: (-int(ticks[e]), int(edges[e, 0]), e))
    for tick in range(8):
        trace.append(v.copy())
        for e in order:
            if tick >= ticks[e]:
                target = int(edges[e, 1]) + 1
                if f32_weights:
                    v[target] = np.float32(v[target] + np.float32(weights[e]))
                else:
                    v[target] = np.float32(np.float64(v[target]) + weights[e])
                events += 1
    return {"edges": edges, "weights": weights, "ticks": ticks, "v": v, "trace": np.asarray(trace), "events": events}


def training_graph_fixture(reset="subtract", detach=True, window=None):
    """The recurrent, tied projection graph of test_native_training_graph.py:19-35: input ->
    hidden, a hidden -> hidden recurrence whose four edges share two parameters, hidden ->
    output and an output -> hidden feedback, with its weights, inputs, labels and initial
    membranes (immediate output spikes make the feedback weights' VJP nonzero)."""
    from atlas_hip import training
    recurrent = dict(source_layer=1, target_layer=1, parameter_count=2, sources=[0, 1, 0, 1], targets=[0, 1, 1, 0],
                     parameter_ids=[0, 0, 1, 1])
    projections = [training.dense_training_projection(0, 1, 2, 2), recurrent,
                   training.dense_training_projection(1, 2, 2, 2), training.dense_training_projection(2, 1, 2, 2)]
    plan = training.lif_training_plan([2, 2, 2], projections=projections, beta=[.5, .75], reset=reset,
                                      detach_reset=detach, surrogate_slope=2, tbptt_window=window)
    weights = [[1.2, .4, .2, 1.1], [.13, -.03], [.8, .2, .3, .9], [.1, -.02, .04, .1]]
    x = np.array([[[1., 0.], [0., 1.], [1., 1.], [0., 1.], [1., 0.], [1., 1.], [0., 1.], [1., 0.]],
                  [[0., 1.], [1., 0.], [1., 1.], [1., 0.], [0., 1.], [1., 0.], [1., 1.], [0., 1.]]])
    initial = np.array([[.3, 1.9, 1.8, 1.7], [1.2, .1, 1.6, 1.9]])
    return plan, weights, x, [0, 1], initial


# ------------------------------------ summed variables and clock-driven synapse states
def summed_pin_network(sources, targets, g0, *, n: int = 4, steps: int = 1, decay: float = 1.0, scale: float = 1.0,
                       dtype: str = "f32", target_range: tuple | None = None, initial: float = 5.0) -> dict:
    """n neurons that never fire (v = 0 < 1) and hold I, J (``dtype``), initially ``initial``; one
    explicit synapse (sources/targets local to the full population and ``target_range``) whose
    state g (``dtype``, initially g0) decays as g <- g * decay each tick (clock-driven), with the
    summed variables I_post = g * scale and J_pre = g * scale."""
    f32 = dtype == "f32"
    w = wide if f32 else (lambda x: x)
    nar = narrow if f32 else (lambda x: x)
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=3)
    full = np.full(n, initial)
    P = b.population("neurongroup", n, states={"v": ("f64", VOLT, np.zeros(n)), "I": (dtype, DIMLESS, full),
                                               "J": (dtype, DIMLESS, full)},
                     parameters={"one": ("f64", VOLT, 1.0)}, threshold=op("gt", ld("v"), ld("one")))
    value = mul(w(ld("g")), ld("scale"))
    b.projection("syn", P, P, on_pre=[stmt("g", dtype, ld("g"))], explicit=(np.asarray(sources), np.asarray(targets)),
                 target_range=target_range, states={"g": (dtype, DIMLESS, np.asarray(g0, np.float64))},
                 parameters={"decay": ("f64", DIMLESS, decay), "scale": ("f64", DIMLESS, scale)},
                 delay_ticks=1, clock_driven=[stmt("g", dtype, nar(mul(w(ld("g")), ld("decay"))))],
                 summed=[("I", value, "post"), ("J", value, "pre")])
    return b.document()


def summed_network(n: int = 20_000, *, indegree: int = 100, steps: int = 300, seed: int = 7, dtype: str = "f32",
                   delay_ticks: int = 1) -> dict:
    """A LIF population (El above threshold, so it fires on its own) whose synaptic current is a
    summed variable: each synapse holds g (clock-driven, g <- g * exp(-dt / 5 ms) every tick; an
    on_pre event adds its weight w ~ U(0, 0.02)) and every neuron's I is, before its update, the
    sum over its incoming edges of g * (E - v_post) with E = -80 mV (Brian2
    ``I_post = g*(E - v_post) : volt (summed)``); J_pre = g * w sums each source's outgoing
    edges.  Fixed in-degree topology, delay ``delay_ticks``."""
    f32 = dtype == "f32"
    w_ = wide if f32 else (lambda x: x)
    nar = narrow if f32 else (lambda x: x)
    rng = np.random.default_rng(seed)
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    Vt, Vr, El = -0.05, -0.06, -0.045
    zeros = np.zeros(n)
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    v = w_(ld("v"))
    update = [stmt("v", dtype, nar(add(v, div(mul(ld("dt"), add(sub(ld("El"), v), w_(ld("I")))), ld("taum")))), VOLT)]
    P = b.population("neurongroup", n,
                     states={"v": (dtype, VOLT, Vr + rng.random(n) * (Vt - Vr)), "I": (dtype, VOLT, zeros),
                             "J": (dtype, DIMLESS, zeros)},
                     parameters={"taum": scalar(0.02, SECOND), "El": scalar(El, VOLT), "Vt": scalar(Vt, VOLT),
                                 "Vr": scalar(Vr, VOLT)},
                     update=([], update), threshold=op("gt", v, ld("Vt")), reset=[stmt("v", dtype, nar(ld("Vr")), VOLT)])
    g = w_(ld("g"))
    b.projection("syn", P, P, on_pre=[stmt("g", dtype, nar(add(g, ld("w"))))], fixed_indegree=indegree,
                 post_aliases={"v_post": "v"}, states={"g": (dtype, DIMLESS, zeros[:0])},
                 parameters={"w": ("f64", DIMLESS, None), "decay": scalar(float(np.exp(-1e-4 / 5e-3)), DIMLESS),
                             "E": scalar(-0.08, VOLT)},
                 initializers={"w": models.initializer_uniform(0.0, 0.02)}, delay_ticks=delay_ticks,
                 clock_driven=[stmt("g", dtype, nar(mul(g, ld("decay"))))],
                 summed=[("I", mul(g, sub(ld("E"), w_(ld("v_post")))), "post"), ("J", mul(g, ld("w")), "pre")])
    doc = b.document()
    # g starts at zero on every edge (the edge count is the rule's)
    syn = doc["instance"]["synapses"][0]
    syn["initial_state"]["g"] = models.hex_array(np.zeros(n * indegree), dtype)
    return protocol.seal(doc)


def summed_multiclock_network(n: int = 4000, *, indegree: int = 40, steps: int = 600, seed: int = 9) -> dict:
    """Two LIF populations on two clocks (A on dt, firing on its own; B on 2 dt) joined by a synapse
    A -> B whose g decays clock-driven on A's clock and jumps by w per event (delay 1): B's current
    is the summed variable g (E - v_post) on B's clock (E = 0, driving B to fire), and J_pre = g w sums each A neuron's edges
    on A's clock.  ``steps`` ticks of A (even)."""
    rng = np.random.default_rng(seed)
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    slow = b.add_clock(2e-4)
    Vt, Vr = -0.05, -0.06
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    pops = []
    for name, el, clock in (("groupA", -0.045, 0), ("groupB", -0.052, slow)):
        zeros = np.zeros(n)
        v = wide(ld("v"))
        update = [stmt("v", "f32", narrow(add(v, div(mul(ld("dt"), add(sub(ld("El"), v), wide(ld("I")))), ld("taum")))),
                       VOLT)]
        pops.append(b.population(
            name, n, states={"v": ("f32", VOLT, Vr + rng.random(n) * (Vt - Vr)), "I": ("f32", VOLT, zeros),
                             "J": ("f32", DIMLESS, zeros)},
            parameters={"taum": scalar(0.02, SECOND), "El": scalar(el, VOLT), "Vt": scalar(Vt, VOLT),
                        "Vr": scalar(Vr, VOLT)},
            update=([], update), threshold=op("gt", v, ld("Vt")), reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)],
            clock=clock))
    g = wide(ld("g"))
    b.projection("syn", pops[0], pops[1], on_pre=[stmt("g", "f32", narrow(add(g, ld("w"))))], fixed_indegree=indegree,
                 post_aliases={"v_post": "v"}, states={"g": ("f32", DIMLESS, np.zeros(0))},
                 parameters={"w": ("f64", DIMLESS, None), "decay": scalar(float(np.exp(-1e-4 / 5e-3)), DIMLESS),
                             "E": scalar(0.0, VOLT)},
                 initializers={"w": models.initializer_uniform(0.0, 0.04)}, delay_ticks=1,
                 clock_driven=[stmt("g", "f32", narrow(mul(g, ld("decay"))))],
                 summed=[("I", mul(g, sub(ld("E"), wide(ld("v_post")))), "post"), ("J", mul(g, ld("w")), "pre")])
    doc = b.document()
    doc["instance"]["synapses"][0]["initial_state"]["g"] = models.hex_array(np.zeros(n * indegree), "f32")
    return protocol.seal(doc)


# ------------------------------------------------------------------------ clocks
def multiclock_network(n: int = 3000, *, steps: int = 600, seed: int = 11, indegree: int = 60,
                       monitor: bool = True, per_edge: bool = False, zero_delay: bool = False) -> dict:
    """Three CUBA populations on three clocks, dt = 0.1 ms, 1.5 dt and 2 dt (the coupled clocks
    of test_gpu_multiclock.py:36-52): fast -> mid with per-edge delays of 1-3 fast ticks, mid ->
    slow with 2 mid ticks, slow -> fast with 1 slow tick (each pathway on its source's clock),
    every population with its state monitor (v of its first 8 neurons) and spike monitor on its own
    clock.  ``steps`` fast ticks (a multiple of 6).  ``per_edge`` gives mid -> slow per-edge
    weights, so its events are delivered in order rather than counted.  ``zero_delay`` gives fast ->
    mid delays of 0-2 ticks and slow -> fast a delay of 0: those events arrive in the tick that
    emitted them."""
    c = models.CUBA
    rng = np.random.default_rng(seed)
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    mid, slow = b.add_clock(1.5e-4), b.add_clock(2e-4)
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    params = {"taum": scalar(c["taum"], SECOND), "taue": scalar(c["taue"], SECOND), "taui": scalar(c["taui"], SECOND),
              "El": scalar(c["El"], VOLT), "Vt": scalar(c["Vt"], VOLT), "Vr": scalar(c["Vr"], VOLT)}
    pops = []
    for k, clock in enumerate((0, mid, slow)):
        m = n // 3
        zeros = np.zeros(m)
        pops.append(b.population(
            f"group{k}", m, states={"v": ("f32", VOLT, c["Vr"] + rng.random(m) * (c["Vt"] - c["Vr"]) * 1.05),
                                    "ge": ("f32", VOLT, zeros), "gi": ("f32", VOLT, zeros)},
            parameters=params, update=models.cuba_update("f32"), threshold=op("gt", wide(ld("v")), ld("Vt")),
            reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=c["refractory"],
            state_monitor=(["v"], list(range(8))) if monitor else None, clock=clock))
    m = n // 3
    plan = ((0, 1, (0, 2)), (1, 2, (2, 2)), (2, 0, (0, 0))) if zero_delay else \
        ((0, 1, (1, 3)), (1, 2, (2, 2)), (2, 0, (1, 1)))
    for k, (s, t, delays) in enumerate(plan):
        src, tgt = models.fixed_indegree_sample(rng, m, m, indegree)
        weight = c["we"] * 3.0 if k < 2 else c["wi"] * 0.5
        if per_edge and k == 1:
            weight = weight * (0.5 + rng.random(src.size))
        state = "ge" if k < 2 else "gi"
        b.projection(f"proj{k}", pops[s], pops[t], on_pre=[stmt(state, "f32", narrow(add(wide(ld(state)), ld("w"))),
                                                               VOLT)],
                     post_aliases={state: state}, parameters={"w": ("f64", VOLT, weight)}, explicit=(src, tgt),
                     delay_ticks=rng.integers(delays[0], delays[1] + 1, src.size))
    return b.document()

def clock_arrival_network(source_clock: int, delay: int, ticks, indices) -> dict:
    """A two-neuron spike generator on one of two clocks (0: dt = 0.1 ms, 60 ticks; 1: dt =
    0.15 ms, 40 ticks) driving one accumulator (v += w, w = 1 and 16 by source) on the other
    clock, with ``delay`` ticks of the source's clock, and a state monitor on v.  With no update
    or threshold the monitored v at each target tick is the sum of the arrivals at earlier
    times."""
    b = NetworkBuilder(dt=1e-4, steps=60, seed=3)
    mid = b.add_clock(1.5e-4)
    clocks = (0, mid)
    gen = b.spike_generator("generator", 2, ticks, indices, clock=clocks[source_clock])
    acc = b.population("accumulator", 1, states={"v": ("f64", VOLT, np.zeros(1))}, state_monitor=(["v"], [0]),
                       clock=clocks[1 - source_clock])
    b.projection("arrivals", gen, acc, on_pre=[stmt("v", "f64", add(ld("v"), ld("w")), VOLT)],
                 post_aliases={"v": "v"}, parameters={"w": ("f64", VOLT, np.array([1.0, 16.0]))},
                 explicit=(np.array([0, 1]), np.array([0, 0])), delay_ticks=np.array([delay, delay]))
    return b.document()


# ------------------------------------------------- recording windows
def window_neuron(steps: int) -> dict:
    """The network of the reference's recording-window test (test_device.py:554-577): one neuron,
    dv/dt = 0 (Euler), threshold v > 0, reset v = 1, v = 1, dt = 1 ms, state and spike monitors,
    recording_window_steps = 3."""
    builder = NetworkBuilder(dt=1e-3, steps=steps, seed=1)
    builder.population("window_group", 1, states={"v": ("f64", DIMLESS, np.ones(1))},
                       update=([], [stmt("v", "f64", ld("v"))]), threshold=op("gt", ld("v"), lit(0.0)),
                       reset=[stmt("v", "f64", lit(1.0))], state_monitor=(["v"], [0]))
    return models.with_recording_window(builder.document(), 3)


def shared_draw_network(n: int = 300, *, steps: int = 200, seed: int = 5, threshold: bool = False) -> dict:
    """Neurons whose update draws once per tick in a scalar statement (``_u = rand()`` on stream 2,
    shared by every neuron: Program::prepare's draw index 0, executor.rs:5488-5503) and once per
    neuron in a vector statement (stream 3): x += _u, y += rand().  With ``threshold`` they also
    fire when y passes 0.5 (reset y = 0), so a shared draw also drives a raster."""
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    zeros = np.zeros(n)
    update = ([stmt("_u", "f64", models.rand(2))],
              [stmt("x", "f64", add(ld("x"), ld("_u"))), stmt("y", "f64", add(ld("y"), mul(models.rand(3), ld("_u"))))])
    kwargs = {}
    if threshold:
        kwargs = {"threshold": op("gt", ld("y"), lit(0.5)), "reset": [stmt("y", "f64", lit(0.0))]}
    b.population("neurongroup", n, states={"x": ("f64", DIMLESS, zeros), "y": ("f64", DIMLESS, zeros)},
                 update=update, frozen=(), **kwargs)
    return b.document()


def log_network(n: int = 2000, *, steps: int = 1000, seed: int = 6) -> dict:
    """Neurons drifting by logarithms of counter-RNG draws (vector log on the device through the
    shared correctly rounded atlas_log): x += log(rand() + 0.25) in f64, y (f32) decays and gains
    log(2 + rand()); a neuron fires when x falls below -20 and x resets to 0."""
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    zeros = np.zeros(n)
    log = lambda e: {"op": "log", "arg": e}  # noqa: E731
    update = ([], [stmt("x", "f64", add(ld("x"), log(add(models.rand(3), lit(0.25))))),
                   stmt("y", "f32", narrow(add(mul(wide(ld("y")), lit(0.999)), log(add(lit(2.0), models.rand(4))))))])
    b.population("neurongroup", n, states={"x": ("f64", DIMLESS, zeros), "y": ("f32", DIMLESS, zeros)},
                 update=update, threshold=op("lt", ld("x"), lit(-20.0)), reset=[stmt("x", "f64", lit(0.0))],
                 frozen=())
    return b.document()


# ------------------------------------------------- run_regularly
def regular_counter(steps: int, *, counter_when: str = "start", with_mid: bool = True) -> dict:
    """Three neurons with f64 states x, y, z, w: the update copies y = x; run_regularly code
    x = x + 1 at `counter_when`, w = y at after_groups (between the update and the threshold
    slot), and z = x + y at the end of the tick.  Closed forms after T ticks: x = T; y = T when the
    counter runs before the update (start), T - 1 when it runs at the end; w = y; z = x + y."""
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=3)
    zeros = np.zeros(3)
    p = b.population("counters", 3, states={s: ("f64", DIMLESS, zeros) for s in ("x", "y", "z", "w")},
                     update=([], [stmt("y", "f64", ld("x"))]), spike_monitor=False)
    b.run_regularly(p, [stmt("x", "f64", add(ld("x"), lit(1.0)))], when=counter_when, name="counter")
    if with_mid:
        b.run_regularly(p, [stmt("w", "f64", ld("y"))], when="after_groups", name="copy")
    b.run_regularly(p, [stmt("z", "f64", add(ld("x"), ld("y")))], when="end", name="total")
    return b.document()


def regular_cuba(n: int, steps: int, *, delay_ticks: int = 1, end: bool = True) -> dict:
    """CUBA (Bernoulli p = 0.02) with run_regularly code at three places: gi decayed by a further
    0.999 at the start of the tick (before the update), v nudged by 10 uV after the update (before
    the threshold), and, with `end`, ge raised by 10 uV at the end of the tick (after the reset)."""
    from atlas_hip.models import narrow, wide
    regular = [("decay_gi", "start", [stmt("gi", "f32", narrow(mul(wide(ld("gi")), lit(0.999))), VOLT)]),
               ("nudge_v", "after_groups", [stmt("v", "f32", narrow(add(wide(ld("v")), lit(1e-5))), VOLT)])]
    if end:
        regular.append(("drive_ge", "end", [stmt("ge", "f32", narrow(add(wide(ld("ge")), lit(1e-5))), VOLT)]))
    return models.cuba_network(n, steps=steps, delay_ticks=delay_ticks, regular=tuple(regular))


# ------------------------------------------------- custom events
def custom_event_network(n: int = 4, *, steps: int = 12, dt: float = 1.0 / 1024, seed: int = 3,
                         scale: int = 1) -> dict:
    """The source group of the reference's custom-event test (test_gpu_custom_events.py:20-40),
    without its event-triggered pathways: dv/dt = 512 Hz (unless refractory), dx/dt = 256 Hz, a
    spike at v >= 1 (reset v = 0, refractory 2 dt), events alpha (x >= 0.5, run_on_event x = 0) and
    zeta (x >= 0.25, run_on_event y += 0.125), x starting at 0 or 0.25; EventMonitors on alpha, spike
    and zeta at the thresholds slot (v, x, y) and on alpha at the end of the tick (x, y).  ``scale``
    repeats the four neurons' initial states (and may offset x) for a larger population."""
    b = NetworkBuilder(dt=dt, steps=steps, seed=seed)
    count = n * scale
    rng = np.random.default_rng(seed)
    x0 = np.tile([0.0, 0.25, 0.0, 0.25], count // 4 + 1)[:count]
    if scale > 1:
        x0 = x0 + rng.random(count) * 0.25
    hz = 1.0
    update = ([], [stmt("v", "f64", add(ld("v"), mul(ld("dt"), mul(lit(512.0), ld("not_refractory"))))),
                   stmt("x", "f64", add(ld("x"), mul(ld("dt"), lit(256.0 * hz))))])
    b.population("source", count,
                 states={"v": ("f64", DIMLESS, np.zeros(count)), "x": ("f64", DIMLESS, x0),
                         "y": ("f64", DIMLESS, np.zeros(count))},
                 update=update, threshold=op("ge", ld("v"), lit(1.0)), reset=[stmt("v", "f64", lit(0.0))],
                 refractory=2 * dt, frozen=(),
                 custom_events={"alpha": (op("ge", ld("x"), lit(0.5)), [stmt("x", "f64", lit(0.0))]),
                                "zeta": (op("ge", ld("x"), lit(0.25)), [stmt("y", "f64", add(ld("y"), lit(0.125)))])},
                 event_monitors=[("alpha", ["v", "x", "y"], "thresholds"), ("spike", ["v", "x", "y"], "thresholds"),
                                 ("zeta", ["v", "x", "y"], "thresholds"), ("alpha", ["x", "y"], "end")])
    return b.document()


def custom_route_network(*, steps: int = 12, delay_shift: int = 0, two_clocks: bool = True,
                         mutable: bool = False, post_delay: int | None = None) -> dict:
    """The network of the reference's custom-event route test (test_gpu_custom_events.py:20-46,
    immutable case): the source group of custom_event_network; a target group (5 neurons, v:1,
    spike at v >= 2 with reset v = 0, event reply at v >= 0.5, on a clock of 2 dt); one Synapses
    from source[1:4] to target[1:5] with edges i = [2, 0, 1, 0, 2], j = [1, 1, 2, 1, 0], w = 0.125
    constant, and three on_pre pathways on three source events: spike_path (v_post += w, delays
    [0, 1, 2, 0, 3] dt), alpha_path (v_post += 2 w, delays [2, 0, 3, 1, 2] dt) and zeta_path
    (v_post += 4 w, delay 0); EventMonitors on the source's events and the target's reply.
    ``delay_shift`` adds ticks to every delay; ``two_clocks`` False puts the target on dt; ``mutable``
    makes w a synapse state that every pathway raises by 0.0625 after its v_post update (the
    reference test's mutable case); ``post_delay`` adds its on_post pathway (w -= 0.03125 on the
    target's reply event) with that delay in ticks (one for all edges, or one per edge)."""
    dt = 1.0 / 1024
    b = NetworkBuilder(dt=dt, steps=steps, seed=5)
    update = ([], [stmt("v", "f64", add(ld("v"), mul(ld("dt"), mul(lit(512.0), ld("not_refractory"))))),
                   stmt("x", "f64", add(ld("x"), mul(ld("dt"), lit(256.0))))])
    source = b.population(
        "source", 4,
        states={"v": ("f64", DIMLESS, np.zeros(4)), "x": ("f64", DIMLESS, np.array([0.0, 0.25, 0.0, 0.25])),
                "y": ("f64", DIMLESS, np.zeros(4))},
        update=update, threshold=op("ge", ld("v"), lit(1.0)), reset=[stmt("v", "f64", lit(0.0))],
        refractory=2 * dt, frozen=(),
        custom_events={"alpha": (op("ge", ld("x"), lit(0.5)), [stmt("x", "f64", lit(0.0))]),
                       "zeta": (op("ge", ld("x"), lit(0.25)), [stmt("y", "f64", add(ld("y"), lit(0.125)))])},
        event_monitors=[("alpha", ["v", "x", "y"], "thresholds"), ("spike", ["v", "x", "y"], "thresholds"),
                        ("zeta", ["v", "x", "y"], "thresholds"), ("alpha", ["x", "y"], "end")],
        state_monitor=(["v", "x", "y"], [0, 1, 2, 3]))
    clock = b.add_clock(2 * dt) if two_clocks else 0
    target = b.population(
        "target", 5, states={"v": ("f64", DIMLESS, np.zeros(5))}, update=None,
        threshold=op("ge", ld("v"), lit(2.0)), reset=[stmt("v", "f64", lit(0.0))], frozen=(),
        spike_monitor=False, custom_events={"reply": (op("ge", ld("v"), lit(0.5)), None)},
        event_monitors=[("reply", ["v"], "thresholds")], state_monitor=(["v"], [0, 1, 2, 3, 4]), clock=clock)
    w = ld("w")
    on_pre = {"alpha_path": [stmt("v_post", "f64", add(ld("v_post"), mul(lit(2.0), w)))],
              "spike_path": [stmt("v_post", "f64", add(ld("v_post"), w))],
              "zeta_path": [stmt("v_post", "f64", add(ld("v_post"), mul(lit(4.0), w)))]}
    if mutable:
        for statements in on_pre.values():
            statements.append(stmt("w", "f64", add(ld("w"), lit(0.0625))))
    shift = np.int64(delay_shift)
    weights = {"states": {"w": ("f64", DIMLESS, np.full(5, 0.125))}} if mutable else \
        {"parameters": {"w": ("f64", DIMLESS, 0.125)}}
    if post_delay is not None:
        weights.update(on_post=[stmt("w", "f64", sub(ld("w"), lit(0.03125)))], post_event="reply",
                       post_delay_ticks=np.asarray(post_delay))
    b.projection("projection", source, target, on_pre=on_pre, source_range=(1, 4), target_range=(1, 5),
                 post_aliases={"v_post": "v"}, **weights,
                 explicit=(np.array([2, 0, 1, 0, 2]), np.array([1, 1, 2, 1, 0])),
                 pre_events={"alpha_path": "alpha", "spike_path": "spike", "zeta_path": "zeta"},
                 delay_ticks={"alpha_path": np.array([2, 0, 3, 1, 2]) + shift,
                              "spike_path": np.array([0, 1, 2, 0, 3]) + shift, "zeta_path": shift})
    return b.document()


def read_events(data: bytes, document: dict) -> tuple[dict, dict]:
    """An events.bin (B2EVT001) read back: ({(population, event): (ticks, indices)},
    {monitor name: (ticks, indices, {variable: values})}), for tests."""
    import struct as _struct
    from atlas_hip.engine import NUMPY
    d = document["definition"]
    assert data[:8] == b"B2EVT001"
    o = 8
    (nstreams,) = _struct.unpack_from("<Q", data, o)
    o += 8
    streams = {}
    keys = [(p, e) for p, pdef in enumerate(d["populations"]) for e in pdef["events"]]
    assert len(keys) == nstreams
    for key in keys:
        (count,) = _struct.unpack_from("<Q", data, o)
        o += 8
        pairs = np.frombuffer(data, "<i8", 2 * count, o).reshape(count, 2)
        o += 16 * count
        streams[key] = (pairs[:, 0].copy(), pairs[:, 1].copy())
    (nmon,) = _struct.unpack_from("<Q", data, o)
    o += 8
    monitors = {}
    for pdef in d["populations"]:
        symbols = {s["name"]: s for s in pdef["states"] + pdef["parameters"]}
        for monitor in pdef.get("event_monitors", []):
            count, nvars = _struct.unpack_from("<QQ", data, o)
            o += 16
            pairs = np.frombuffer(data, "<i8", 2 * count, o).reshape(count, 2)
            o += 16 * count
            values = {}
            for name in monitor["variables"]:
                dt = np.dtype(NUMPY[symbols[name]["dtype"]]).newbyteorder("<")
                values[name] = np.frombuffer(data, dt, count, o).copy()
                o += dt.itemsize * count
            monitors[monitor["name"]] = (pairs[:, 0].copy(), pairs[:, 1].copy(), values)
    assert len(monitors) == nmon and data[o:o + 8] == b"B2EEND01"
    return streams, monitors


def custom_only_network(steps: int = 6, *, record: bool = True, dt: float = 1.0 / 1024) -> dict:
    """The reference's custom-only population (test_gpu_custom_events.py:63-70): two neurons, dv/dt =
    512 Hz, events crossing (v >= 1, run_on_event v = 0; z += 0.25) and quiet (never), no spike
    event and no synapse; with ``record`` an EventMonitor on crossing at the end of the tick."""
    b = NetworkBuilder(dt=dt, steps=steps, seed=1)
    update = ([], [stmt("v", "f64", add(ld("v"), mul(ld("dt"), lit(512.0))))])
    b.population("neurongroup", 2, states={"v": ("f64", DIMLESS, np.zeros(2)), "z": ("f64", DIMLESS, np.zeros(2))},
                 update=update, frozen=(), spike_monitor=False,
                 custom_events={"crossing": (op("ge", ld("v"), lit(1.0)),
                                             [stmt("v", "f64", lit(0.0)), stmt("z", "f64", add(ld("z"), lit(0.25)))]),
                                "quiet": ({"op": "boolean", "value": False}, None)},
                 event_monitors=[("crossing", ["v", "z"], "end")] if record else None)
    return b.document()


def custom_cuba_network(n: int = 4000, *, steps: int = 2000, delay_ticks: int = 1, seed: int = 4,
                        routes: tuple | None = None, counted: bool = False) -> dict:
    """CUBA neurons (El above the threshold, so they fire on their own) driven by a spike generator
    (as generator_network) with a custom event "high" (v > -50.5 mV, run_on_event ge = ge / 2) beside
    the spike, EventMonitors on high at the threshold
    (v, ge) and at the end of the tick (ge), and on the spike at the end (v).  ``routes`` = (lo, hi)
    adds a recurrent Synapses (in-degree 20) with two on_pre pathways: high_path on the high event
    (gi -= 0.05 mV, per-edge delays lo..hi ticks) and spike_path on the spike (ge += 0.2 mV, delay
    lo); ``counted`` gives that Synapses a state c (f64) that high_path raises by 1 and spike_path
    multiplies by 1.5, so both pathways touch the same records in an order that matters."""
    c = models.CUBA
    rng = np.random.default_rng(seed)
    n_inputs = 500
    keys = rng.choice(steps * n_inputs, size=min(20_000, steps * n_inputs), replace=False)
    b = NetworkBuilder(dt=1e-4, steps=steps, seed=seed)
    G = b.spike_generator("spikegeneratorgroup", n_inputs, keys // n_inputs, keys % n_inputs)
    zeros = np.zeros(n)
    scalar = lambda value, dims: ("f64", dims, value)  # noqa: E731
    P = b.population(
        "neurongroup", n,
        states={"v": ("f32", VOLT, c["Vr"] + rng.random(n) * (c["Vt"] - c["Vr"])), "ge": ("f32", VOLT, zeros),
                "gi": ("f32", VOLT, zeros)},
        parameters={"taum": scalar(c["taum"], SECOND), "taue": scalar(c["taue"], SECOND),
                    "taui": scalar(c["taui"], SECOND), "El": scalar(-45e-3, VOLT),
                    "Vt": scalar(c["Vt"], VOLT), "Vr": scalar(c["Vr"], VOLT)},
        update=models.cuba_update("f32"), threshold=op("gt", wide(ld("v")), ld("Vt")),
        reset=[stmt("v", "f32", narrow(ld("Vr")), VOLT)], refractory=c["refractory"],
        custom_events={"high": (op("gt", wide(ld("v")), lit(-0.0505)),
                                [stmt("ge", "f32", narrow(div(wide(ld("ge")), lit(2.0))), VOLT)])},
        event_monitors=[("high", ["v", "ge"], "thresholds"), ("high", ["ge"], "end"), ("spike", ["v"], "end")])
    src, tgt = models.fixed_indegree_sample(rng, n_inputs, n, 40)
    b.projection("synapses", G, P, on_pre=[stmt("ge", "f32", narrow(add(wide(ld("ge")), ld("w"))), VOLT)],
                 post_aliases={"ge": "ge"}, parameters={"w": ("f64", VOLT, 3.0e-3)}, explicit=(src, tgt),
                 delay_ticks=delay_ticks)
    if routes is not None:
        lo, hi = routes
        src, tgt = models.fixed_indegree_sample(rng, n, n, 20)
        on_pre = {"high_path": [stmt("gi", "f32", narrow(sub(wide(ld("gi")), ld("wi"))), VOLT)],
                  "spike_path": [stmt("ge", "f32", narrow(add(wide(ld("ge")), ld("we"))), VOLT)]}
        states = {}
        if counted:
            on_pre["high_path"].append(stmt("c", "f64", add(ld("c"), lit(1.0))))
            on_pre["spike_path"].append(stmt("c", "f64", mul(ld("c"), lit(1.5))))
            states = {"c": ("f64", DIMLESS, np.zeros(src.size))}
        b.projection("recurrent", P, P, post_aliases={"ge": "ge", "gi": "gi"}, on_pre=on_pre, states=states,
                     pre_events={"high_path": "high"},
                     parameters={"wi": ("f64", VOLT, 5.0e-5), "we": ("f64", VOLT, 2.0e-4)}, explicit=(src, tgt),
                     delay_ticks={"high_path": rng.integers(lo, hi + 1, src.size), "spike_path": lo})
    return b.document()
