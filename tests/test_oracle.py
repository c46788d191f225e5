"""Pins of the CPU oracle (oracle/): the reference's golden data, published
closed forms, the reference's own invariants and independent evaluations.

The oracle is the checker of every GPU parity test, so each of its parts is
tied here to something outside it:

* executor semantics, delayed delivery, refractory and the dump format: the
  reference-produced dump of ``tests/fixtures/reference-v1`` (byte-exact);
* both ``mix64`` variants: the published splitmix64 output sequence;
* Floyd fixed in-degree and fixed-total topologies: the invariants of
  large_topology.rs:399-419 and uniformity of the chosen subsets;
* delivery chronology: the same-tick three-delay KAT of test_metal_delays.py;
* Euler update, threshold, refractory, delayed delivery and reset order: an
  independent dense f64 evaluation of the reference's recurrent workload
  with its acceptance tolerances (gpu_recurrent.py:29-31);
* the README single-neuron example (9 spikes) and its closed-form period;
* summed variables and clock-driven synapse states (executor.rs:2513-2597):
  f32 sums whose value depends on edge order and per-addition rounding, the
  zero fill of the endpoint range, closed-form decays, and exact dyadic sums
  equal to per-endpoint totals;
* several clocks (executor.rs:3940-3964): arrival times across clocks of 0.1
  and 0.15 ms written out in integer units, coincident ticks included.
"""
import json
import math

import numpy as np
import pytest

import nets
from atlas_hip import models, protocol, results
from oracle import oracle

SPLITMIX_SEED0 = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
SPLITMIX_SEED1234567 = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431]
GOLDEN_GAMMA = 0x9E3779B97F4A7C15
MASK = (1 << 64) - 1


@pytest.fixture(scope="module", autouse=True)
def _built():
    oracle.build()


def test_reference_golden_dump_byte_exact(golden):
    model = json.loads((golden / "reference_v1_model.json").read_text())
    out = oracle.run(model)
    assert out.results == (golden / "reference_v1_results.bin").read_bytes()
    assert out.events == (golden / "reference_v1_events.bin").read_bytes()
    summary = json.loads((golden / "reference_v1_summary.json").read_text())
    assert out.spike_count == summary["spike_count"] == 155
    assert out.synaptic_events == summary["synaptic_events"] == 1238


def test_golden_dump_detects_a_changed_delay(golden):
    """The golden comparison is sensitive to delivery timing: one pathway's delays moved by a tick change the dump."""
    model = json.loads((golden / "reference_v1_model.json").read_text())
    pathway = model["instance"]["synapses"][0]["pathways"][0]
    pathway["delay_ticks"] = [d + 1 for d in pathway["delay_ticks"]]
    protocol.seal(model)
    out = oracle.run(model)
    assert out.results != (golden / "reference_v1_results.bin").read_bytes()


def _uniform53(value: int) -> float:
    return (value >> 11) * 2.0 ** -53


def test_counter_rng_is_splitmix64_finaliser():
    """counter_uniform (executor.rs:190-207): mix64 without the gamma pre-add of the counter.
    counter = seed ^ stream*C1 ^ ..., so seed = k*gamma reproduces splitmix64's k-th output."""
    state = 0
    for k, expected in enumerate(SPLITMIX_SEED0, start=1):
        state = (state + GOLDEN_GAMMA) & MASK
        assert oracle.counter_uniform(state, 0, 0, 0) == _uniform53(expected)
    assert oracle.counter_uniform(0, 0, 0, 0) == 0.0
    # stream * 0x9e3779b97f4a7c15 with stream = 1 lands on the same counter as seed = gamma
    assert oracle.counter_uniform(0, 1, 0, 0) == _uniform53(SPLITMIX_SEED0[0])
    state = 1234567
    for expected in SPLITMIX_SEED1234567:
        state = (state + GOLDEN_GAMMA) & MASK
        assert oracle.counter_uniform(state, 0, 0, 0) == _uniform53(expected)


def test_pathway_draws_are_indexed_by_edge_and_delivery_tick():
    """A pathway's rand() draws counter_uniform(seed, stream, tick, edge) (executor.rs:5071-5074,
    5572-5577): the iteration domain active_synapses binds the edge index of the projection's own
    edge order, at the tick the event is delivered.  Pinned against a direct evaluation of the
    pinned counter_uniform over the run's deliveries in the canonical order (ticks ascending, fired
    sources ascending, each source's edges ascending), accumulated in f64 as the program does; the
    edges are listed shuffled, so indexing by the sorted row, by the target or by the spike's
    tick instead gives other sums."""
    from atlas_hip import engine as eng
    from atlas_hip.results import read_results
    doc = models.random_pathway_network(60, 80, spikes=400, indegree=6, steps=120, delay_ticks=2)
    plan = eng.lower(doc)
    got = read_results(oracle.run(doc).results, plan.document).populations[1].states[0]
    path = plan.pathways[0]
    _, src, tgt = path.topology
    schedule = doc["instance"]["populations"][0]["spike_generator"]
    fired: dict = {}
    for t, i in zip(schedule["spike_ticks"], schedule["spike_indices"]):
        fired.setdefault(t, []).append(i)
    edges_of = [np.flatnonzero(src == s) for s in range(60)]

    def expected(index, tick_of):
        x = np.zeros(80)
        for arrival in range(plan.steps):
            for s in sorted(fired.get(arrival - 2, [])):
                for e in edges_of[s]:
                    x[tgt[e]] += oracle.counter_uniform(plan.rng_seed, 1, tick_of(arrival), index(e))
        return x

    np.testing.assert_array_equal(got, expected(lambda e: e, lambda t: t))
    rows = np.empty(src.size, np.int64)
    rows[np.lexsort((np.arange(src.size), tgt, src))] = np.arange(src.size)
    assert not np.array_equal(got, expected(lambda e: rows[e], lambda t: t))
    assert not np.array_equal(got, expected(lambda e: tgt[e], lambda t: t))
    assert not np.array_equal(got, expected(lambda e: e, lambda t: t - 2))


def test_scalar_draws_take_index_zero_once_per_tick():
    """A scalar statement's rand() is drawn once per tick with draw index 0 (Program::prepare,
    executor.rs:5488-5503: scalar_random_bindings) and shared by every neuron, a vector statement's
    per neuron: x += _u and y += rand() _u equal their direct evaluation over the ticks; a draw
    indexed by the neuron in the scalar statement, or at the previous tick, gives other values."""
    from atlas_hip import engine as eng
    from atlas_hip.results import read_results
    doc = nets.shared_draw_network(40, steps=60)
    plan = eng.lower(doc)
    x, y = read_results(oracle.run(doc).results, plan.document).populations[0].states
    ticks = range(plan.start_tick, plan.start_tick + plan.steps)

    def expected(index, shift):
        ex, ey = np.zeros(40), np.zeros(40)
        for t in ticks:
            for i in range(40):
                u = oracle.counter_uniform(plan.rng_seed, 2, t - shift, index(i))
                ex[i] = ex[i] + u
                ey[i] = ey[i] + oracle.counter_uniform(plan.rng_seed, 3, t, i) * u
        return ex, ey

    ex, ey = expected(lambda i: 0, 0)
    np.testing.assert_array_equal(x, ex)
    np.testing.assert_array_equal(y, ey)
    assert not np.array_equal(x, expected(lambda i: i, 0)[0])
    assert not np.array_equal(x, expected(lambda i: 0, 1)[0])


def test_custom_events_follow_their_closed_forms():
    """Named events beside the spike (executor.rs:4098-4118, 4157-4186; the reference's own
    test_gpu_custom_events.py:20-70 network): x gains 0.25 per tick, alpha (x >= 0.5) resets it to
    0, zeta (x >= 0.25) adds 0.125 to y, v gains 0.5 per tick outside a refractory tick.  So alpha
    fires on alternate ticks by the neuron's starting x, zeta at every tick, the spike every third
    tick from tick 1; the end-of-tick monitor sees x = 0 (the reference test's own check) and
    y = 0.125 (t + 1); zeta outnumbers the spikes.  A custom-only population's crossing event
    (v >= 1, then v = 0 and z += 0.25) fires every other tick."""
    from atlas_hip import engine as eng
    doc = nets.custom_event_network()
    streams, monitors = nets.read_events(oracle.run(doc).events, doc)
    ticks = np.arange(12)
    spike_t, spike_i = streams[(0, "spike")]
    assert sorted(zip(spike_t, spike_i)) == [(t, i) for t in range(1, 12, 3) for i in range(4)]
    alpha = sorted(zip(*streams[(0, "alpha")]))
    assert alpha == sorted((t, i) for t in ticks for i in range(4) if (t + i) % 2 == 1)
    assert sorted(zip(*streams[(0, "zeta")])) == [(t, i) for t in ticks for i in range(4)]
    t_end, i_end, values = monitors["source_alpha_end_eventmonitor3"]
    assert sorted(zip(t_end, i_end)) == alpha
    np.testing.assert_array_equal(values["x"], 0.0)
    np.testing.assert_array_equal(values["y"], 0.125 * (t_end + 1))
    assert len(monitors["source_zeta_thresholds_eventmonitor2"][0]) > len(spike_t)
    t_thr, _, values = monitors["source_alpha_thresholds_eventmonitor0"]
    np.testing.assert_array_equal(values["x"], 0.5)
    np.testing.assert_array_equal(values["y"], 0.125 * t_thr)
    only = nets.custom_only_network()
    streams, monitors = nets.read_events(oracle.run(only).events, only)
    assert sorted(zip(*streams[(0, "crossing")])) == [(t, i) for t in (1, 3, 5) for i in range(2)]
    assert len(streams[(0, "quiet")][0]) == 0
    t_end, _, values = next(iter(monitors.values()))
    np.testing.assert_array_equal(values["v"], 0.0)
    np.testing.assert_array_equal(values["z"], 0.25 * (t_end + 1) / 2)
    assert eng.lower(only).populations[0].custom_events


def test_custom_event_routes_follow_the_source_events():
    """Pathways triggered by the source's spike, alpha and zeta events (the reference's route test,
    test_gpu_custom_events.py:20-46, immutable case), replayed by hand from the source events'
    closed forms (spike at ticks 1, 4, 7, 10; alpha where t + i is odd; zeta every tick): an
    event of neuron i at tick t adds coef * w to v of each edge's target at tick t + delay, in the
    synapses slot; the target (clock 2 dt) samples v at the start of its ticks, fires spike
    (v >= 2, reset to 0 after the tick's deliveries) and reply (v >= 0.5) at its thresholds, which
    precede the same step's deliveries.  With the delays shifted by a tick, on one clock, and with
    w a synapse state every pathway raises by 0.0625 after its update of v_post (pathways of one
    step in name order: alpha, spike, zeta), and an on_post pathway on the target's reply event
    lowering w by 0.03125 on each in-edge after the step's on_pre pathways (one delay, or the
    reference test's per-edge on_post delays, counted in the target's ticks: with the target on
    2 dt this is the reference test's mutable case whole)."""
    from atlas_hip.results import read_results
    edges = [(2, 1), (0, 1), (1, 2), (0, 1), (2, 0)]   # (source - 1, target - 1), local indices
    for shift, two, mutable, post in ((0, True, False, None), (1, True, False, None), (0, False, False, None),
                                      (2, False, False, None), (0, True, True, None), (1, False, True, None),
                                      (0, False, True, 0), (1, False, True, 2), (0, False, True, [0, 1, 2, 1, 3]),
                                      (1, False, True, [2, 0, 1, 3, 1]), (0, True, True, [0, 1, 2, 1, 3])):
        doc = nets.custom_route_network(delay_shift=shift, two_clocks=two, mutable=mutable, post_delay=post)
        res = oracle.run(doc)
        events = {"spike": [(t, i) for t in range(1, 12, 3) for i in range(4)],
                  "alpha": [(t, i) for t in range(12) for i in range(4) if (t + i) % 2 == 1],
                  "zeta": [(t, i) for t in range(12) for i in range(4)]}
        routes = {"alpha": ([2, 0, 3, 1, 2], 2.0), "spike": ([0, 1, 2, 0, 3], 1.0), "zeta": ([0] * 5, 4.0)}
        arrivals = {}   # tick -> [(pathway rank, edge, coef)]
        for rank, (event, (delays, coef)) in enumerate(routes.items()):
            for t, i in events[event]:
                for e, ((a, j), d) in enumerate(zip(edges, delays)):
                    if a + 1 == i:
                        arrivals.setdefault(t + d + shift, []).append((rank, e, coef))
        step = 2 if two else 1
        v, w, samples, spikes, reply = np.zeros(5), np.full(5, 0.125), [], [], []
        for t in range(12):
            mine = t % step == 0
            if mine:
                samples.append(v.copy())
                fired = [j for j in range(5) if v[j] >= 2.0]
                reply += [(t // step, j) for j in range(5) if v[j] >= 0.5]
                spikes += [(t // step, j) for j in fired]
            for _, e, coef in sorted(arrivals.get(t, [])):
                v[edges[e][1] + 1] += coef * w[e]
                if mutable:
                    w[e] += 0.0625
            if post is not None and mine:
                # on_post after the step's on_pre pathways, on the target's clock: each in-edge of a
                # neuron whose reply fired the edge's delay (in target ticks) ago
                post_delays = np.broadcast_to(np.asarray(post), (5,))
                for tick, j in reply:
                    for e, (_, jj) in enumerate(edges):
                        if jj + 1 == j and tick == t // step - post_delays[e]:
                            w[e] -= 0.03125
            if mine:
                v[fired] = 0.0
        dump = read_results(res.results, doc)
        target = dump.populations[1]
        np.testing.assert_array_equal(target.states[0], v)
        if mutable:
            np.testing.assert_array_equal(dump.synapses[0]["states"][0], w)
        np.testing.assert_array_equal(target.samples[0], np.array(samples))
        streams, _ = nets.read_events(res.events, doc)
        assert sorted(zip(*streams[(1, "spike")])) == sorted(spikes)
        assert sorted(zip(*streams[(1, "reply")])) == sorted(reply)
        assert spikes and reply


def test_poisson_group_fires_at_its_rates():
    """The oracle's PoissonGroup threshold (rand() < rates * dt on the counter RNG): each
    neuron's spike count over 4000 ticks is Binomial(4000, rate * dt); the total lies within
    5 standard deviations of its mean, and fast neurons fire more than slow ones."""
    from atlas_hip import engine as eng
    from atlas_hip.results import read_results
    doc = models.poisson_network(400, 50, indegree=10, steps=4000, rates=(5.0, 80.0))
    result = oracle.run(doc)
    plan = eng.lower(doc)
    spikes = read_results(result.results, plan.document).populations[0].spikes
    counts = np.bincount(spikes[:, 1], minlength=400)
    rates = plan.populations[0].vector_params["rates"][1]
    p = rates * 1e-4
    mean, sd = (4000 * p).sum(), np.sqrt((4000 * p * (1 - p)).sum())
    assert abs(counts.sum() - mean) < 5 * sd, (counts.sum(), mean, sd)
    slow, fast = counts[rates < 20].mean(), counts[rates > 60].mean()
    assert fast > 3 * slow


def test_spike_generator_emits_its_schedule():
    """A SpikeGeneratorGroup's raster is its schedule (executor.rs:3008-3036: at each tick the
    scheduled neurons, ascending); a synchronous volley at tick 10 reaches every target of the
    inputs one tick later; a schedule out of order or outside the run is rejected."""
    from atlas_hip import engine as eng
    from atlas_hip.results import read_results
    from oracle.ir_compile import UnsupportedModel
    doc = models.generator_network(200, 300, spikes=3000, indegree=20, steps=400)
    result = oracle.run(doc)
    plan = eng.lower(doc)
    dump = read_results(result.results, plan.document)
    schedule = doc["instance"]["populations"][0]["spike_generator"]
    raster = dump.populations[0].spikes
    np.testing.assert_array_equal(raster[:, 0], schedule["spike_ticks"])
    np.testing.assert_array_equal(raster[:, 1], schedule["spike_indices"])
    assert np.count_nonzero(raster[:, 0] == 10) == 200
    bad = json.loads(json.dumps(doc, default=str))
    gen = bad["instance"]["populations"][0]["spike_generator"]
    gen["spike_ticks"][0], gen["spike_ticks"][1] = gen["spike_ticks"][1] + 1, gen["spike_ticks"][0]
    with pytest.raises(UnsupportedModel):
        oracle.run(bad)


def test_event_monitor_records_spikes_with_values_before_the_reset():
    """An EventMonitor on the spike event (executor.rs:3053-3080) at the thresholds slot: its events
    are the spike raster, each recorded v lies above the threshold (read after the update, before
    the reset), and a scalar parameter is recorded as its value."""
    import struct
    from atlas_hip import engine as eng
    from atlas_hip.results import read_results
    doc = models.cuba_network(500, steps=600, event_monitor=["v", "ge", "Vt"])
    result = oracle.run(doc)
    plan = eng.lower(doc)
    raster = read_results(result.results, plan.document).populations[0].spikes
    ev = result.events
    off = 16 + sum(0 for _ in ())
    for _ in range(struct.unpack_from("<Q", ev, 8)[0]):
        off += 8 + 16 * struct.unpack_from("<Q", ev, off)[0]
    assert struct.unpack_from("<Q", ev, off)[0] == 1
    n, nvars = struct.unpack_from("<QQ", ev, off + 8)
    assert n == len(raster) > 50 and nvars == 3
    pairs = np.frombuffer(ev, "<i8", 2 * n, off + 24).reshape(n, 2)
    np.testing.assert_array_equal(pairs, raster)
    base = off + 24 + 16 * n
    v = np.frombuffer(ev, "<f4", n, base)
    vt = np.frombuffer(ev, "<f8", n, base + 8 * n)
    assert np.all(v > -50e-3) and np.all(vt == -50e-3)
    assert ev.endswith(b"B2EEND01")


def test_topology_rng_is_splitmix64():
    """uniform_open (large_topology.rs:54-75): mix64 with the gamma pre-add, edge * gamma in the counter,
    so edge k of seed 0 is splitmix64(seed 0)'s (k+1)-th output; value = (m + 0.5) * 2^-53."""
    values = oracle.uniform(4, 0, 0, 0.0, 1.0)
    for k, expected in enumerate(SPLITMIX_SEED0):
        assert values[k] == ((expected >> 11) + 0.5) * 2.0 ** -53
    scaled = oracle.uniform(4, 0, 0, 2.0, 6.0)
    np.testing.assert_array_equal(scaled, 2.0 + 4.0 * values)


def test_fixed_indegree_reference_invariants():
    """large_topology.rs:399-419: distinct sources per target, source-major order, reproducible, seed-sensitive."""
    src, tgt = oracle.fixed_indegree(11, 7, 5, 123)
    again = oracle.fixed_indegree(11, 7, 5, 123)
    np.testing.assert_array_equal(src, again[0])
    np.testing.assert_array_equal(tgt, again[1])
    assert src.size == 35
    assert np.all(np.diff(src.astype(np.int64)) >= 0)
    for target in range(7):
        assert len(set(src[tgt == target].tolist())) == 5
    other = oracle.fixed_indegree(11, 7, 5, 124)
    assert not (np.array_equal(src, other[0]) and np.array_equal(tgt, other[1]))
    with pytest.raises(oracle.OracleError):
        oracle.fixed_indegree(4, 2, 5, 1)


def test_fixed_indegree_targets_ascend_within_a_source():
    src, tgt = oracle.fixed_indegree(50, 300, 20, 9)
    key = src.astype(np.int64) * 1000 + tgt
    assert np.all(np.diff(key) > 0)
    assert np.array_equal(np.bincount(tgt, minlength=300), np.full(300, 20))


def test_fixed_indegree_subsets_are_uniform():
    """Floyd's algorithm draws every K-subset with equal probability: each source is chosen with
    probability K/N and each pair with K(K-1)/(N(N-1)).  A wrong draw bound or index skews these."""
    n, k, targets = 9, 3, 60000
    src, tgt = oracle.fixed_indegree(n, targets, k, 77)
    counts = np.bincount(src, minlength=n)
    expected = targets * k / n
    chi2 = float(((counts - expected) ** 2 / expected).sum())
    assert chi2 < 30.0, chi2           # 8 dof; p ~ 2e-4
    order = np.argsort(tgt, kind="stable")
    per_target = np.sort(src[order].reshape(targets, k), axis=1)
    full = np.zeros((n, n), np.int64)
    for a, b in ((0, 1), (0, 2), (1, 2)):
        np.add.at(full, (per_target[:, a], per_target[:, b]), 1)
    upper = full[np.triu_indices(n, 1)]
    expected_pair = targets * 3 / (n * (n - 1) / 2)
    chi2 = float(((upper - expected_pair) ** 2 / expected_pair).sum())
    assert chi2 < 80.0, chi2           # 35 dof; p ~ 2e-5


def test_fixed_total_reference_invariants():
    src, tgt = oracle.fixed_total(5, 7, 10000, 123)
    again = oracle.fixed_total(5, 7, 10000, 123)
    np.testing.assert_array_equal(src, again[0])
    np.testing.assert_array_equal(tgt, again[1])
    assert np.all(np.diff(src.astype(np.int64)) >= 0)
    assert src.max() < 5 and tgt.max() < 7
    other = oracle.fixed_total(5, 7, 10000, 124)
    assert not (np.array_equal(src, other[0]) and np.array_equal(tgt, other[1]))


def test_chronology_kat():
    doc = nets.chronology_kat()
    out = oracle.run(doc)
    dump = results.read_results(out.results, doc)
    np.testing.assert_array_equal(dump.populations[1].states[0], np.array([1.0, 0.0], np.float32))
    assert out.synaptic_events == 3
    np.testing.assert_array_equal(dump.populations[0].spikes, [[0, 1], [1, 2], [2, 0]])


def test_readme_lif_nine_spikes():
    doc = nets.readme_lif()
    out = oracle.run(doc)
    assert out.spike_count == 9
    dump = results.read_results(out.results, doc)
    # brute force: the same Euler recurrence, one neuron
    v, spikes, ticks = 0.0, 0, []
    for tick in range(1000):
        v = v + 1e-4 * (1.5 - v) / 10e-3
        if v > 1.0:
            spikes += 1
            ticks.append(tick)
            v = 0.0
    assert spikes == 9
    np.testing.assert_array_equal(dump.populations[0].spikes[:, 0], ticks)
    # closed form of the Euler map: v_n = 1.5 (1 - (1 - dt/tau)^n) first exceeds 1 at n = ceil(ln 3 / -ln(1 - dt/tau))
    period = math.floor(math.log(1 / 3) / math.log(1 - 0.01)) + 1
    assert np.all(np.diff(ticks) == period) and ticks[0] == period - 1


@pytest.mark.parametrize("neurons,degree,steps", [(400, 50, 2000), (200, 100, 1500)])
def test_recurrent_workload_against_independent_reference(neurons, degree, steps):
    """Acceptance of gpu_recurrent.py:29-31: exact spike ticks and indices, v within rtol 1e-4, atol 5e-6."""
    doc = nets.recurrent_network(neurons, degree, steps)
    out = oracle.run(doc)
    dump = results.read_results(out.results, doc)
    ref = nets.recurrent_reference(neurons, degree, steps)
    pop = dump.populations[0]
    assert ref["ticks"].size > neurons  # the network is active
    np.testing.assert_array_equal(pop.spikes[:, 0], ref["ticks"])
    np.testing.assert_array_equal(pop.spikes[:, 1], ref["indices"])
    np.testing.assert_allclose(pop.states[0].astype(np.float64), ref["v"], rtol=1e-4, atol=5e-6)
    np.testing.assert_allclose(pop.states[1].astype(np.float64), ref["I_syn"], rtol=1e-4, atol=5e-6)


# ------------------------------------------------------------ shared exponential
def _exact(fn: str, values):
    from decimal import Decimal, getcontext
    getcontext().prec = 60
    out = []
    for v in values:
        d = Decimal(float(v))
        e = d.exp()
        out.append(float(e if fn == "exp" else (e - 1) if fn == "expm1" else (e - 1) / d))
    return np.array(out)


@pytest.mark.parametrize("fn,lo,hi", [("exp", -40.0, 40.0), ("exp", -700.0, 700.0), ("expm1", -2.0, 2.0),
                                      ("expm1", -0.0054, 0.0054), ("expm1", -40.0, 40.0), ("exprel", -20.0, 20.0)])
def test_shared_exponential_is_correctly_rounded(fn, lo, hi):
    """atlas_math.h (shared by the GPU kernels and the oracle) against exactly rounded values
    (60-digit decimal arithmetic).  exprel divides the rounded expm1 by x, as the reference does."""
    x = np.random.default_rng(11).uniform(lo, hi, 3000)
    shared, libm = oracle.math(fn, x)
    if fn == "exprel":
        expm1_shared, _ = oracle.math("expm1", x)
        np.testing.assert_array_equal(shared, expm1_shared / x)
        return
    np.testing.assert_array_equal(shared, _exact(fn, x))
    # the host libm agrees except where it is not correctly rounded (one ulp)
    assert np.abs(shared.view(np.int64) - libm.view(np.int64)).max() <= 1


def test_shared_exponential_special_values():
    x = np.array([0.0, -0.0, 1e-300, -1e-300, 709.78, 709.7827128933840, 709.79, 800.0, -745.0, -746.0, np.inf,
                  -np.inf, np.nan])
    exp_, libm = oracle.math("exp", x)
    np.testing.assert_array_equal(exp_, libm)
    em1, libm1 = oracle.math("expm1", x)
    np.testing.assert_array_equal(em1, libm1)
    assert np.signbit(em1[1]) and em1[0] == 0.0


def test_hh_update_against_independent_reference():
    """The exponential-Euler HH statement trees (models.hh_update) with float64 states against the
    independent f64 evaluation of gpu_hh.py:59-89 (equilibrium/expm1 form): exact spikes, states to 1e-9."""
    doc = nets.hh_ionic_network(200, 10000, dtype="f64")
    out = oracle.run(doc)
    dump = results.read_results(out.results, doc)
    ref = nets.hh_reference(200, 10000)
    pop = dump.populations[0]
    assert ref["ticks"].size > 10000
    np.testing.assert_array_equal(pop.spikes[:, 0], ref["ticks"])
    np.testing.assert_array_equal(pop.spikes[:, 1], ref["indices"])
    for k, name in enumerate(["v", "m", "n", "h", "ge", "gi"]):
        np.testing.assert_allclose(pop.states[k], ref[name], rtol=1e-9, atol=1e-15, err_msg=name)


def test_hh_float32_states_keep_the_reference_raster():
    """With float32 storage (the configs' dtype) the raster still equals the f64 reference over 3000 ticks,
    and the gating variables stay within the acceptance of gpu_hh.py:49."""
    doc = nets.hh_ionic_network(64, 3000)
    dump = results.read_results(oracle.run(doc).results, doc)
    ref = nets.hh_reference(64, 3000)
    pop = dump.populations[0]
    np.testing.assert_array_equal(pop.spikes[:, 0], ref["ticks"])
    np.testing.assert_array_equal(pop.spikes[:, 1], ref["indices"])
    for k, name in enumerate(["v", "m", "n", "h", "ge", "gi"]):
        atol = nets.HH_ACCEPT["atol"][name] * (5 if name == "v" else 1)  # v: float32 storage of a 100 mV swing
        np.testing.assert_allclose(pop.states[k].astype(np.float64), ref[name], rtol=nets.HH_ACCEPT["rtol"],
                                   atol=atol, err_msg=name)


def test_cobahh_is_insensitive_to_the_exponential_implementation():
    """Config 2 with float32 states: the host libm and the shared exponential give identical dumps
    (f32 storage rounding absorbs their rare one-ulp f64 differences)."""
    from atlas_hip import models
    doc = models.cobahh_network(4000, steps=1000)
    a = oracle.run(doc)
    b = oracle.run(doc, shared_math=True)
    assert a.spike_count > 5000
    assert a.results == b.results and a.events == b.events


@pytest.mark.parametrize("neurons,degree,steps", [(64, 8, 400), (256, 16, 1500)])
def test_stdp_workload_against_independent_reference(neurons, degree, steps):
    """The reference's delayed recurrent STDP workload (on_pre delays 0-3, on_post delay 2,
    event-driven traces) against an independent ordered event recurrence (the method of
    gpu_stdp_compare.py:90-117); acceptance of gpu_stdp_compare.py:74 (exact spikes and
    lastupdate, rtol 2e-5 / atol 2e-6 otherwise)."""
    doc = nets.stdp_network(neurons, degree, steps)
    out = oracle.run(doc)
    dump = results.read_results(out.results, doc)
    ref = nets.stdp_reference(neurons, degree, steps)
    pop = dump.populations[0]
    np.testing.assert_array_equal(pop.spikes[:, 0], ref["ticks"])
    np.testing.assert_array_equal(pop.spikes[:, 1], ref["indices"])
    np.testing.assert_allclose(pop.states[0], ref["v"], rtol=2e-5, atol=2e-6)
    syn = dump.synapses[0]
    for k, name in enumerate(["w", "Apre", "Apost", "lastupdate"]):
        if name == "lastupdate":
            np.testing.assert_array_equal(syn["states"][k], ref[name])
        else:
            np.testing.assert_allclose(syn["states"][k], ref[name], rtol=2e-5, atol=2e-6, err_msg=name)
    assert np.unique(ref["lastupdate"]).size > 3


def _segmented(document: dict, boundary: int):
    """(continuous run, second segment of the run split at `boundary`), both oracle results,
    and the number of pending events carried over the boundary."""
    from atlas_hip.continuation import continuation, first_segment
    doc = protocol.load(document)
    steps = int(doc["run"]["clocks"][0]["steps"])
    full = oracle.run(document, shared_math=True, lift_recording_budget=True)
    first_doc = first_segment(document, boundary)
    first = oracle.run(first_doc, shared_math=True, lift_recording_budget=True)
    second_doc = continuation(first_doc, results.result_from_dump(first.results, protocol.load(first_doc)),
                              steps - boundary)
    second = oracle.run(second_doc, shared_math=True, lift_recording_budget=True)
    carried = sum(len(pw["pending"]) for sin in second_doc["instance"]["synapses"] for pw in sin["pathways"])
    return (full, results.read_results(full.results, doc), first,
            second, results.read_results(second.results, protocol.load(second_doc)), carried)


@pytest.mark.parametrize("model,boundary", [
    ("reference", 128),
    ("cuba_delay3", 200),
    ("plastic", 705),
    ("stdp", 200),
    ("cuba_indegree", 150),
])
def test_segmented_run_equals_the_continuous_run(golden, model, boundary):
    """AtlasIR.md section 6 and device.py:2200-2370: a run split in two, the second segment
    carrying final states, refractory state, synapse states and the pending delayed events
    over the boundary, ends bit-identical to the continuous run.  The reference fixture has
    per-edge delays 1-4, the cuba network a uniform delay of 3 ticks, the plastic network STDP
    with per-edge delays 1-20 across a burst, the STDP ring an on_post pathway delayed 2 ticks."""
    document = {"reference": lambda: json.loads((golden / "reference_v1_model.json").read_text()),
                "cuba_delay3": lambda: models.cuba_network(1000, steps=400, delay_ticks=3),
                "cuba_indegree": lambda: models.cuba_network(5000, indegree=100, delay_ticks=3, weight_scale=0.35,
                                                             steps=300),
                "plastic": lambda: models.plastic_network(2000, steps=1000, packed=False),
                "stdp": lambda: nets.stdp_network(64, 8, 400)}[model]()
    full, a, first, second, b, carried = _segmented(document, boundary)
    assert carried > 0
    for pa, pb in zip(a.populations, b.populations):
        assert np.array_equal(pa.spikes[pa.spikes[:, 0] >= boundary], pb.spikes)
        for x, y in zip(pa.states, pb.states):
            assert np.array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8))
        if pa.lastspike is not None:
            assert np.array_equal(pa.lastspike, pb.lastspike)
            assert np.array_equal(pa.not_refractory, pb.not_refractory)
    for sa, sb in zip(a.synapses, b.synapses):
        for x, y in zip(sa["states"], sb["states"]):
            assert np.array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8))
    assert first.synaptic_events + second.synaptic_events == full.synaptic_events


def test_pending_events_are_validated():
    """model.rs:4322-4338: pending events ascend in delivery tick, fall inside the run and
    name an endpoint (uniform delay) or an edge (per-edge delays)."""
    from oracle.ir_compile import UnsupportedModel, compile_model
    base = protocol.load(models.cuba_network(200, steps=50, delay_ticks=3), verify_envelope=False)
    base.pop("protocol", None)
    for pending in ([{"delivery_tick": 5, "item": 0}, {"delivery_tick": 4, "item": 1}],
                    [{"delivery_tick": 50, "item": 0}],
                    [{"delivery_tick": 3, "item": 10_000}]):
        doc = json.loads(json.dumps(base))
        doc["instance"]["synapses"][0]["pathways"][0]["pending"] = pending
        with pytest.raises(UnsupportedModel):
            compile_model(protocol.seal(doc))
    doc = json.loads(json.dumps(base))
    doc["instance"]["synapses"][0]["pathways"][0]["pending"] = [{"delivery_tick": 3, "item": 0},
                                                                {"delivery_tick": 3, "item": 7}]
    compile_model(protocol.seal(doc))


@pytest.mark.parametrize("model", ["reference_example", "weighted_cuba"])
def test_binary_csr_equals_the_explicit_topology(tmp_path, model):
    """A B2CSR001 topology (binary_topology.rs:24-130, executor.rs:35-57) runs exactly as the
    same edges given inline: the oracle's file reader against its explicit path.  The
    reference's conformance model (test_binary_topology.py:19-98) fires neuron 3 at tick 0
    (v0 = 1.1 > 1), whose one edge (to neuron 0, multiplicity 5) arrives two ticks later; the
    other neurons stay below threshold for 2 ms (Euler towards 1.2 with tau = 10 ms)."""
    if model == "reference_example":
        doc, _ = models.binary_csr_example()
    else:
        doc = nets.weighted_cuba()
    binary = models.to_binary_csr(doc, 0, tmp_path / "graph.b2csr")
    assert binary["instance"]["synapses"][0]["topology"]["kind"] == "binary_csr"
    a = oracle.run(doc, shared_math=True)
    b = oracle.run(binary, shared_math=True)
    assert a.results == b.results and a.synaptic_events == b.synaptic_events
    if model == "reference_example":
        dump = results.read_results(a.results, protocol.load(doc))
        assert dump.populations[0].spikes.tolist() == [[0, 3]] and a.synaptic_events == 1
        v = np.linspace(0.0, 1.1, 4)
        for tick in range(20):
            v = v + 1e-4 * (1.2 - v) / 10e-3
            if tick == 0:
                v[3] = 0.0
            if tick == 2:
                v[0] += 0.02 * 5.0
        np.testing.assert_allclose(dump.populations[0].states[0], v, rtol=1e-13)
    else:
        assert a.synaptic_events > 5000


@pytest.mark.parametrize("corruption", ["offsets", "target", "nan", "truncated", "checksum", "header"])
def test_malformed_binary_csr_is_rejected(tmp_path, corruption):
    """The reference's corruptions (test_binary_topology.py:46-58) and a digest mismatch
    (a valid edit, :88-96) fail both the oracle and the engine before anything runs."""
    import struct as struct_
    from atlas_hip import binary_topology, engine
    from oracle.ir_compile import UnsupportedModel, compile_model
    doc, _ = models.binary_csr_example()
    path = tmp_path / "graph.b2csr"
    binary = models.to_binary_csr(doc, 0, path)
    header = binary_topology.HEADER.size
    edits = {"offsets": (header + 8, struct_.pack("<Q", 9)), "target": (header + 5 * 8, struct_.pack("<I", 4)),
             "nan": (header + 5 * 8 + 5 * 4, struct_.pack("<d", float("nan"))),
             "checksum": (header + 5 * 8 + 5 * 4, struct_.pack("<d", 9.0)),
             "header": (8, struct_.pack("<Q", 5))}
    if corruption == "truncated":
        path.write_bytes(path.read_bytes()[:-1])
    else:
        at, data = edits[corruption]
        with path.open("r+b") as stream:
            stream.seek(at)
            stream.write(data)
    if corruption != "checksum":
        # keep the declared digest in step with the edit, so the structural check is the one that fails
        inner = protocol.load(binary, verify_envelope=False)
        inner.pop("protocol", None)
        inner["instance"]["synapses"][0]["topology"]["sha256"] = binary_topology.file_sha256(path)
        binary = protocol.seal(inner)
    with pytest.raises(UnsupportedModel):
        compile_model(binary)
    with pytest.raises(engine.UnsupportedModel):
        engine.lower(binary)


def _poisson_input_population(n: int, count: int, rate: float, steps: int) -> dict:
    """A population of n accumulators x (f64, no dynamics) driven by one PoissonInput
    x += binomial(count, rate dt) * 1 per tick."""
    builder = models.NetworkBuilder(dt=1e-4, steps=steps, seed=99)
    pop = builder.population("inputs", n, states={"x": ("f64", models.DIMLESS, np.zeros(n))}, spike_monitor=False)
    builder.poisson_input(pop, "x", count, rate, 1.0)
    return builder.document()


@pytest.mark.parametrize("count,rate", [(20, 100.0), (1000, 500.0)])
def test_poisson_input_increments_are_binomial(count, rate):
    """A PoissonInput (export.py:571-608) adds binomial(N, rate dt) per tick and neuron
    (counter_binomial, executor.rs:224-268): by inversion when N p <= 5 (N = 20, p = 0.01:
    integers with the Binomial(20, 0.01) frequencies), else its normal approximation
    (N = 1000, p = 0.05: mean N p, variance N p (1 - p), not integer-valued).  Sums over 40
    ticks have mean 40 N p and variance 40 N p (1 - p).  Checked within 5 sigma."""
    import math as math_
    n, p = 20000, rate * 1e-4
    one = results.read_results(oracle.run(_poisson_input_population(n, count, rate, 1), shared_math=True).results,
                               protocol.load(_poisson_input_population(n, count, rate, 1)))
    x = np.asarray(one.populations[0].states[0])
    mean, var = count * p, count * p * (1 - p)
    assert abs(x.mean() - mean) < 5 * math_.sqrt(var / n)
    assert abs(x.var() - var) < 5 * var * math_.sqrt(2.0 / n) + 1e-12
    if count * p <= 5:
        assert np.all(x == np.round(x)) and x.min() >= 0
        observed = np.bincount(x.astype(np.int64), minlength=4)[:3]
        expected = [n * math_.comb(count, k) * p ** k * (1 - p) ** (count - k) for k in range(3)]
        for o, e in zip(observed, expected):
            assert abs(o - e) < 5 * math_.sqrt(e) + 1
    else:
        assert np.mean(x != np.round(x)) > 0.99
    doc = _poisson_input_population(4000, count, rate, 40)
    total = np.asarray(results.read_results(oracle.run(doc, shared_math=True).results, protocol.load(doc))
                       .populations[0].states[0])
    assert abs(total.mean() - 40 * mean) < 5 * math_.sqrt(40 * var / 4000)


def test_counter_normal_draws_are_standard_normal():
    """randn() (counter_normal, executor.rs:200-222: the polar method on pairs of the stream's
    uniform draws): 20,000 accumulators x += randn() over 40 ticks have mean 0 and variance
    40; one tick's draws have variance 1 and fourth moment 3 (a normal's), within 5 sigma."""
    builder = models.NetworkBuilder(dt=1e-4, steps=1, seed=5)
    pop = builder.population("x", 20000, states={"x": ("f64", models.DIMLESS, np.zeros(20000))},
                             update=([], [models.stmt("x", "f64", models.add(models.ld("x"), {"op": "randn", "stream": 3}))]),
                             spike_monitor=False)
    doc = builder.document()
    x = np.asarray(results.read_results(oracle.run(doc, shared_math=True).results, protocol.load(doc))
                   .populations[0].states[0])
    n = x.size
    assert abs(x.mean()) < 5 / math.sqrt(n) and abs(x.var() - 1) < 5 * math.sqrt(2 / n)
    assert abs(np.mean(x ** 4) - 3) < 5 * math.sqrt(96 / n)
    assert np.unique(x).size == n


@pytest.mark.parametrize("lam", [3.0, 50.0])
def test_counter_poisson_draws(lam):
    """poisson(lambda) (counter_poisson, executor.rs:290-323): the product method below 10 and
    PTRS above give integer draws with mean and variance lambda (5 sigma over 20,000 neurons)."""
    builder = models.NetworkBuilder(dt=1e-4, steps=1, seed=5)
    draw = {"op": "poisson", "stream": 4, "lambda": models.ld("lam")}
    builder.population("x", 20000, states={"x": ("f64", models.DIMLESS, np.zeros(20000))},
                       parameters={"lam": ("f64", models.DIMLESS, lam)},
                       update=([], [models.stmt("x", "f64", models.add(models.ld("x"), draw))]), spike_monitor=False)
    doc = builder.document()
    x = np.asarray(results.read_results(oracle.run(doc, shared_math=True).results, protocol.load(doc))
                   .populations[0].states[0])
    n = x.size
    assert np.all(x == np.round(x)) and x.min() >= 0
    assert abs(x.mean() - lam) < 5 * math.sqrt(lam / n)
    assert abs(x.var() - lam) < 5 * lam * math.sqrt((2 + 1 / lam) / n)


# ------------------------------------- procedural topology: the reference's own restatement
@pytest.mark.parametrize("kind", ["total", "indegree"])
def test_procedural_edges_equal_the_reference_test_restatement(kind):
    """Floyd fixed in-degree and fixed total against ``draw``/``endpoints`` of
    test_gpu_initialization.py:29-60 (8 sources -> 5 targets, seed 0x12345678): exact."""
    expected = nets.initialization_endpoints(kind)
    if kind == "total":
        src, tgt = oracle.fixed_total(8, 5, 257, nets.INIT_SEED)
    else:
        src, tgt = oracle.fixed_indegree(8, 5, 3, nets.INIT_SEED)
    np.testing.assert_array_equal(src, expected[:, 0])
    np.testing.assert_array_equal(tgt, expected[:, 1])


def test_initializers_equal_the_reference_test_restatement():
    """materialize_uniform / materialize_clipped_normal against ``uniform``/``normal`` of
    test_gpu_initialization.py:39-47 and 82-88 (streams 2 and 4): exact, with the host libm
    (the reference's Rust f64::ln / cos and the test's math.log / math.cos)."""
    count = 257
    uniform = oracle.uniform(count, nets.INIT_SEED, 2, .0625, .25)
    np.testing.assert_array_equal(uniform, [.0625 + .1875 * nets.initialization_uniform(2, e) for e in range(count)])
    normal = oracle.clipped_normal(count, nets.INIT_SEED, 2, .125, .03, .0625, .25)
    np.testing.assert_array_equal(normal, [nets.initialization_normal(2, e, .125, .03, .0625, .25)
                                           for e in range(count)])
    delays = oracle.clipped_normal(count, nets.INIT_SEED, 4, 1.5, .5, 0.0, 3.0)
    np.testing.assert_array_equal(delays, [nets.initialization_normal(4, e, 1.5, .5, 0, 3) for e in range(count)])
    # with tighter bounds the rejection loop runs (a third of the first draws fall outside)
    tight = oracle.clipped_normal(count, nets.INIT_SEED, 4, 1.5, .5, 1.0, 2.0)
    np.testing.assert_array_equal(tight, [nets.initialization_normal(4, e, 1.5, .5, 1.0, 2.0) for e in range(count)])
    unclipped = oracle.clipped_normal(count, nets.INIT_SEED, 4, 1.5, .5)
    assert np.sum(unclipped != tight) > count // 5


@pytest.mark.parametrize("kind,distribution", [("total", "uniform"), ("total", "normal"),
                                               ("indegree", "uniform"), ("indegree", "normal")])
def test_procedural_network_equals_the_reference_test(kind, distribution):
    """The whole model of test_gpu_initialization.py:63-101 through the oracle: per-edge weights
    and delay initializers, floor(delay/dt + 0.5) quantisation (executor.rs:86-90) and delivery
    in (delay descending, source, edge) order.  The final v and the trace equal the test's loop
    with the CPU engine's arithmetic bit for bit, and its float32 formula within 1 ulp."""
    doc = nets.initialization_network(kind, distribution)
    out = oracle.run(doc)
    dump = results.read_results(out.results, doc)
    exp = nets.initialization_expected(kind, distribution)
    target = dump.populations[1]
    np.testing.assert_array_equal(target.states[0], exp["v"])
    np.testing.assert_array_equal(target.samples[0], exp["trace"])
    assert out.synaptic_events == exp["events"]
    f32 = nets.initialization_expected(kind, distribution, f32_weights=True)
    np.testing.assert_allclose(target.states[0], f32["v"], rtol=2e-7, atol=0)
    assert np.unique(exp["ticks"]).size >= 3  # several delay groups, so the delivery order matters


# ------------------------------------------------------------------ shared logarithm
def _exact_log(values):
    from decimal import Decimal, getcontext
    getcontext().prec = 60
    return np.array([float(Decimal(float(v)).ln()) for v in values])


@pytest.mark.parametrize("lo,hi,scale", [(1e-300, 1e300, "log"), (0.5, 2.0, "lin"), (0.9, 1.1, "lin"),
                                         (1 - 1e-6, 1 + 1e-6, "lin"), (0.0, 1.0, "lin"),
                                         (5e-324, 2.2250738585072014e-308, "lin")])
def test_shared_log_is_correctly_rounded(lo, hi, scale):
    """atlas_log (used by counter_normal, counter_binomial, counter_poisson and the training
    losses) against exactly rounded values (60-digit decimal ln), 3000 arguments per range,
    including the neighbourhood of 1 and subnormals; glibc's log differs by at most one ulp."""
    rng = np.random.default_rng(13)
    x = np.exp(rng.uniform(np.log(lo), np.log(hi), 3000)) if scale == "log" else rng.uniform(lo, hi, 3000)
    x = x[x > 0]
    shared, libm = oracle.math("log", x)
    np.testing.assert_array_equal(shared, _exact_log(x))
    assert np.abs(shared.view(np.int64) - libm.view(np.int64)).max() <= 1


def test_shared_log_special_values_and_halley_regression():
    """Special values equal glibc's; the inputs where the earlier Halley iteration lost up to
    64,561 ulp (x just below 1, where x - e^y cancels) are exactly rounded."""
    x = np.array([0.0, -0.0, -1.0, np.inf, -np.inf, np.nan, 1.0, 2.0, 0.5, 5e-324, 1.7976931348623157e308])
    shared, libm = oracle.math("log", x)
    np.testing.assert_array_equal(shared, libm)
    near = np.array([0.9999945, 1 - 2.0**-53, 1 + 2.0**-52, 0.99, 0.95, 1.0000001])
    shared, _ = oracle.math("log", near)
    np.testing.assert_array_equal(shared, _exact_log(near))


def test_counter_normal_pairing_equals_the_reference_test():
    """counter_normal (executor.rs:206-221) against the pairing convention restated by
    test_gpu_random.py:85-101: pair = index / 2, draws d and d + 1 on the pair's counter,
    the even index takes x1 and the odd one x2, rejection in steps of two draws.  The test's
    own float32 formula (24-bit uniforms) agrees within its tolerance rtol = atol = 3e-6;
    the f64 polar formula with the oracle's counter draws agrees exactly."""
    seed, stream, tick = 1729, 5, 0

    def u24(index, draw):
        x = seed ^ ((stream * 0x9E3779B97F4A7C15) & MASK) ^ ((tick * 0xD1B54A32D192ED03) & MASK)
        x ^= ((index * 0x94D049BB133111EB) & MASK) ^ ((draw * 0x369DEA0F31A53F85) & MASK)
        x = ((x ^ (x >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        x = ((x ^ (x >> 27)) * 0x94D049BB133111EB) & MASK
        return np.float32(((x ^ (x >> 31)) >> 40) / 2**24)

    expected = []
    for pair in range(512):
        for draw in range(0, 8192, 2):
            a = np.float32(2 * u24(pair, draw) - 1)
            c = np.float32(2 * u24(pair, draw + 1) - 1)
            radius = np.float32(a * a + c * c)
            if 0 < radius < 1:
                factor = np.float32(np.sqrt(np.float32(-2 * np.log(radius) / radius)))
                expected.extend([np.float32(factor * a), np.float32(factor * c)])
                break
    actual = np.array([oracle.counter_normal(seed, stream, tick, i) for i in range(1024)])
    np.testing.assert_allclose(actual, expected, rtol=3e-6, atol=3e-6)
    shared = np.array([oracle.counter_normal(seed, stream, tick, i, shared=True) for i in range(1024)])
    np.testing.assert_array_equal(shared, actual)


# ------------------------------------ summed variables and clock-driven synapse states
def _pin_states(doc):
    dump = results.read_results(oracle.run(doc).results, doc)
    v, i_sum, j_sum = (np.asarray(x, np.float64) for x in dump.populations[0].states)
    return i_sum, j_sum, np.asarray(dump.synapses[0]["states"][0], np.float64)


@pytest.mark.parametrize("dtype,values,expected", [
    ("f32", [1.0, 2.0**-24, 2.0**-24], 1.0),             # each 1 + 2^-24 ties to even: 1
    ("f32", [2.0**-24, 2.0**-24, 1.0], 1.0 + 2.0**-23),  # 2^-23 first, then exact
    ("f64", [1.0, 2.0**-24, 2.0**-24], 1.0 + 2.0**-23)])
def test_summed_variable_adds_in_edge_order_rounding_each_addition(dtype, values, expected):
    """A summed variable adds each edge's value in edge order and an f32 state rounds after
    every addition (add_f64, executor.rs:517-523): 1 + 2^-24 + 2^-24 stays 1 in f32 but the
    reverse order, or an f64 state, reaches 1 + 2^-23.  Neurons without edges are set to 0."""
    i_sum, j_sum, _ = _pin_states(nets.summed_pin_network([0, 1, 2], [3, 3, 3], values, dtype=dtype))
    assert i_sum.tolist() == [0.0, 0.0, 0.0, expected]
    assert j_sum.tolist() == [*values, 0.0]


def test_summed_variable_fills_only_its_endpoint_range():
    """The target range [2, 4): its neuron without edges becomes 0, neurons outside it keep
    their value (fill_f64 over target_start..target_start + target_count, executor.rs:2557)."""
    i_sum, j_sum, _ = _pin_states(nets.summed_pin_network([0, 1], [1, 1], [0.25, 0.5], target_range=(2, 4)))
    assert i_sum.tolist() == [5.0, 5.0, 0.0, 0.75]
    assert j_sum.tolist() == [0.25, 0.5, 0.0, 0.0]


def test_clock_driven_decay_and_summed_order_closed_form():
    """g <- g / 2 every tick from g0 = (1, 3): after T = 10 ticks g = g0 2^-10 exactly, and the
    last tick's summed variable (order -1, before the state update of order 0 in the groups
    slot) saw g0 2^-9, replacing rather than accumulating the previous ticks' sums."""
    i_sum, _, g = _pin_states(nets.summed_pin_network([0, 2], [1, 1], [1.0, 3.0], decay=0.5, steps=10))
    assert g.tolist() == [2.0**-10, 3 * 2.0**-10]
    assert i_sum.tolist() == [0.0, 4 * 2.0**-9, 0.0, 0.0]


def test_summed_dyadic_sums_equal_endpoint_totals():
    """Multiples of 2^-8 below 4 sum exactly in f32: every target's I and every source's J
    equal the totals over its edges (numpy bincount), whatever the order."""
    rng = np.random.default_rng(5)
    n, edges = 16, 60
    src, tgt = rng.integers(0, n, edges), rng.integers(0, n, edges)
    g0 = rng.integers(0, 1024, edges) / 256.0
    i_sum, j_sum, _ = _pin_states(nets.summed_pin_network(src, tgt, g0, n=n, scale=2.0))
    assert np.array_equal(i_sum, 2 * np.bincount(tgt, g0, n))
    assert np.array_equal(j_sum, 2 * np.bincount(src, g0, n))


@pytest.mark.parametrize("source_clock,delay,ticks,indices", [
    (1, 2, [0, 5, 37, 38], [0, 1, 0, 1]),
    (0, 3, [0, 10, 56, 57], [0, 1, 0, 1])])
def test_multiclock_arrivals_follow_the_merged_steps(source_clock, delay, ticks, indices):
    """Clocks of 0.1 and 0.15 ms: a spike at source tick T arrives at source tick T + delay (the
    pathway runs on its source's clock) if that tick is within the source's run.  The target's
    monitor at its tick k, which runs before the synapses slot of its step, has seen exactly the
    arrivals at earlier times, so one at the same time as k (0.3 ms = 3 x 0.1 = 2 x 0.15, which
    differ in their last bits and share a step by the epsilon rule) is seen from k + 1.  The
    final v holds every delivered arrival, also those after the target's last tick.  In units
    of 0.05 ms the two dts are 2 and 3."""
    doc = nets.clock_arrival_network(source_clock, delay, ticks, indices)
    dump = results.read_results(oracle.run(doc).results, doc)
    units = (2, 3)
    src_units, tgt_units = units[source_clock], units[1 - source_clock]
    src_steps, tgt_steps = (60, 40)[source_clock], (60, 40)[1 - source_clock]
    weights = (1.0, 16.0)
    arrivals = [(t + delay, weights[i]) for t, i in zip(ticks, indices) if t + delay < src_steps]
    assert len(arrivals) == 3
    trace = dump.populations[1].samples[0][:, 0]
    expected = [sum(w for a, w in arrivals if a * src_units < k * tgt_units) for k in range(tgt_steps)]
    assert trace.tolist() == expected
    assert dump.populations[1].states[0].tolist() == [sum(w for _, w in arrivals)]
    assert dump.synapses[0]["delivered"] == 3
    # the coincident arrival is seen one target tick after its time
    first = arrivals[0][0] * src_units // tgt_units
    assert arrivals[0][0] * src_units == first * tgt_units and expected[first] == 0 and expected[first + 1] == 1.0
    # the generator's spikes are recorded in its own clock's ticks
    assert sorted(map(tuple, dump.populations[0].spikes.tolist())) == sorted(zip(ticks, indices))


# ------------------------------------------------------------------ recording windows
def test_recording_window_bounds_monitors_across_runs():
    """test_device.py:554-577: a 5-tick run with a 3-tick window records the states and spikes of
    ticks 2, 3, 4 (count 3); the next 5-tick run records ticks 7, 8, 9 (count 3 again)."""
    from atlas_hip.continuation import continuation
    doc = nets.window_neuron(5)
    assert doc["definition"]["populations"][0]["monitor"]["window_steps"] == 3
    out = oracle.run(doc)
    pop = results.read_results(out.results, doc).populations[0]
    assert pop.spikes[:, 0].tolist() == [2, 3, 4] and pop.counts.tolist() == [3]
    assert pop.samples[0].shape == (3, 1) and pop.samples[0].ravel().tolist() == [1.0, 1.0, 1.0]
    following = continuation(doc, results.result_from_dump(out.results, doc), 5)
    assert following["run"]["clocks"][0]["start_tick"] == 5
    assert following["definition"]["populations"][0]["monitor"]["window_steps"] == 3
    pop = results.read_results(oracle.run(following).results, following).populations[0]
    assert pop.spikes[:, 0].tolist() == [7, 8, 9] and pop.counts.tolist() == [3]
    assert pop.samples[0].shape == (3, 1)


@pytest.mark.parametrize("window", [1, 700, 1999])
def test_recording_window_keeps_the_last_ticks_of_the_full_run(window):
    """CUBA 1000 over 2000 ticks with a state monitor of 20 neurons: the windowed run's spikes are
    the full run's at ticks >= 2000 - window, its counts those spikes' counts, its samples the
    full run's last `window` rows, and its final states, last spikes and event counts equal the
    full run's (the window changes what is recorded, not the dynamics)."""
    record = list(range(0, 1000, 50))
    full_doc = models.cuba_network(1000, steps=2000, state_monitor=(["v", "ge"], record))
    doc = models.with_recording_window(full_doc, window)
    full = results.read_results(oracle.run(full_doc).results, full_doc)
    part = results.read_results(oracle.run(doc).results, doc)
    a, b = full.populations[0], part.populations[0]
    keep = a.spikes[:, 0] >= 2000 - window
    assert np.array_equal(b.spikes, a.spikes[keep]) and len(b.spikes) > 0 or window == 1
    assert np.array_equal(b.counts, np.bincount(a.spikes[keep, 1], minlength=1000))
    for x, y in zip(a.samples, b.samples):
        assert y.shape == (window, len(record)) and np.array_equal(y, x[-window:])
    assert np.array_equal(a.last_fired, b.last_fired) and np.array_equal(a.lastspike, b.lastspike)
    for x, y in zip(a.states, b.states):
        assert np.array_equal(x, y)
    assert full.synapses[0]["delivered"] == part.synapses[0]["delivered"]


# ------------------------------------------------------------------ run_regularly
@pytest.mark.parametrize("counter_when,y_offset", [("start", 0), ("end", 1)])
def test_run_regularly_runs_at_its_schedule_slot(counter_when, y_offset):
    """run_regularly code runs over every neuron at its node (executor.rs:4139-4148): x = x + 1
    at the start of each tick precedes the update y = x (y = T after T ticks); at the end of the
    tick it follows it (y = T - 1).  w = y after the update copies this tick's y; z = x + y at the
    end sees both."""
    T = 37
    doc = nets.regular_counter(T, counter_when=counter_when)
    pop = results.read_results(oracle.run(doc).results, doc).populations[0]
    x, y, z, w = (np.asarray(a) for a in pop.states)
    assert np.all(x == T) and np.all(y == T - y_offset) and np.all(w == y) and np.all(z == x + y)


def test_run_regularly_places_in_the_tick():
    """The engine's place of each run_regularly node: before the update (start), between the update
    and the threshold (after_groups), after the reset (end); own clocks and reads of
    not_refractory before the update are rejected."""
    from atlas_hip import engine
    plan = engine.lower(nets.regular_counter(5))
    assert [(c["name"], where) for c, where in plan.populations[0].regular] == [
        ("counter", "pre"), ("copy", "mid"), ("total", "end")]
    plan = engine.lower(nets.regular_cuba(400, 20, end=False))
    assert [where for _, where in plan.populations[0].regular] == ["pre", "mid"]
    doc = nets.regular_cuba(400, 20)
    pre = doc["definition"]["populations"][0]["code_objects"][-3]
    assert pre["name"] == "decay_gi"
    pre["vector"][0]["value"] = models.narrow(models.mul(models.wide(models.ld("gi")), models.ld("not_refractory")))
    pre["effects"]["reads"].append("not_refractory")
    protocol.seal(doc)
    with pytest.raises(engine.UnsupportedModel, match="not_refractory"):
        engine.lower(doc)
    doc = nets.regular_counter(5)
    next(c for c in doc["definition"]["populations"][0]["code_objects"] if c["name"] == "counter")["clock"] = 1
    protocol.seal(doc)
    with pytest.raises(engine.UnsupportedModel, match="own clock"):
        engine.lower(doc)
