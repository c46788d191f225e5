"""GPU parity: the HIP engine (through libatlas_sim_hip.so) against the reference's
golden dump and the CPU oracle, on the same AtlasIR documents.

Bar: spike rasters, counts, last-spike lists, refractory state and synaptic event
counts bit-exact; states bit-exact (both paths evaluate f64 registers with f32
storage rounding per statement, so the results are identical, not merely close).
"""
import struct

import numpy as np
import pytest

import nets
from atlas_hip import engine, models
from atlas_hip.executor import HipExecutor
from atlas_hip.results import read_results, write_events, write_results
from oracle import oracle

pytestmark = pytest.mark.gpu


def run_gpu(doc, **kwargs):
    with HipExecutor(doc, device=0, **kwargs) as ex:
        result = ex.run()
        return ex.document, result, write_results(ex.document, result), write_events(ex.document, result)


def assert_same_dump(document, got: bytes, expected: bytes):
    if got == expected:
        return
    a, b = read_results(got, document), read_results(expected, document)
    for k, (pa, pb) in enumerate(zip(a.populations, b.populations)):
        assert np.array_equal(pa.spikes, pb.spikes), f"population {k}: spike raster differs"
        for s, (x, y) in enumerate(zip(pa.states, pb.states)):
            assert np.array_equal(x, y), f"population {k} state {s} differs (max |d|={np.max(np.abs(x - y))})"
    for k, (sa, sb) in enumerate(zip(a.synapses, b.synapses)):
        assert sa["delivered"] == sb["delivered"], f"synapse {k}: delivered {sa['delivered']} != {sb['delivered']}"
    raise AssertionError("dumps differ in bytes outside spikes/states/delivered")


def test_reference_fixture_byte_exact(golden):
    print("case: reference-v1 fixture", flush=True)
    doc, result, dump, events = run_gpu(golden / "reference_v1_model.json")
    assert_same_dump(doc, dump, (golden / "reference_v1_results.bin").read_bytes())
    assert events == (golden / "reference_v1_events.bin").read_bytes()
    assert sum(len(p["spike_ticks"]) for p in result["populations"]) == 155
    assert sum(s["events"] for s in result["synapses"]) == 1238


@pytest.mark.parametrize("n,steps", [(1000, 400), (4000, 2000)])
def test_cuba_bernoulli_matches_oracle(n, steps):
    print(f"case: CUBA bernoulli n={n} steps={steps}", flush=True)
    doc = models.cuba_network(n, steps=steps)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    assert expected.spike_count > 0 and expected.synaptic_events > 0


@pytest.mark.parametrize("delay", [1, 3])
def test_scaled_cuba_fixed_indegree_matches_oracle(delay):
    print(f"case: scaled CUBA fixed indegree delay={delay}", flush=True)
    doc = models.cuba_network(20000, indegree=100, delay_ticks=delay, steps=300, weight_scale=0.8)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


def test_replay_is_deterministic():
    print("case: replay determinism", flush=True)
    doc = models.cuba_network(3000, steps=600)
    with HipExecutor(doc, device=0) as ex:
        first = write_results(ex.document, ex.run())
        second = write_results(ex.document, ex.run())
    assert first == second


def test_burst_overflows_lds_staging():
    """Every neuron fires at tick 0; tick 1 delivers ~1M events per 1024-target block,
    far beyond the 4096-event LDS staging buffer, so delivery flushes many times."""
    print("case: synchronous burst, multi-flush delivery", flush=True)
    from atlas_hip import protocol
    from atlas_hip.models import hex_array
    doc = models.cuba_network(2048, indegree=1024, delay_ticks=1, steps=40, weight_scale=0.01)
    doc["instance"]["populations"][0]["initial_state"]["v"] = hex_array(np.full(2048, -0.0495), "f32")
    protocol.seal(doc)
    expected = oracle.run(doc)
    assert expected.synaptic_events >= 2048 * 1024
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


def test_voltage_jump_synapses_unfused_reset():
    """on_pre writes v like the reset does: deliveries into two delay slots, the
    inhibitory pathway ordered after the excitatory one on the same state, and the
    reset running after the deliveries."""
    print("case: delta LIF, shared post state, unfused reset", flush=True)
    doc = models.delta_lif_network(6000, indegree=200, steps=1500)
    expected = oracle.run(doc)
    assert expected.spike_count > 1000
    with HipExecutor(doc, device=0) as ex:
        assert not ex.plan.populations[0].reset_fused
        assert [len(g) for g in ex.plan.groups] == [1, 1]
        result = ex.run()
        dump, events = write_results(ex.document, result), write_events(ex.document, result)
    assert_same_dump(ex.document, dump, expected.results)
    assert events == expected.events


def test_chronology_kat():
    """test_metal_delays.py:49-93 re-expressed: three same-tick arrivals from delays 0, 1, 2 apply in
    emission order (float32 sums 2**24, 0, 1), so target v = [1, 0]."""
    print("case: delivery chronology KAT", flush=True)
    doc = nets.chronology_kat()
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    np.testing.assert_array_equal(result["populations"][1]["states"]["v"], np.array([1.0, 0.0], np.float32))
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


def test_readme_lif():
    print("case: README single LIF neuron", flush=True)
    doc = nets.readme_lif()
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert len(result["populations"][0]["spike_ticks"]) == 9
    assert_same_dump(document, dump, expected.results)


def test_recurrent_workload():
    """The reference's recurrent comparison workload: bit-exact with the oracle, and within the
    acceptance of gpu_recurrent.py:29-31 (exact spikes, rtol 1e-4, atol 5e-6) of the independent
    f64 evaluation."""
    print("case: recurrent CUBA workload 400x50, 2000 ticks", flush=True)
    doc = nets.recurrent_network(400, 50, 2000)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    ref = nets.recurrent_reference(400, 50, 2000)
    pop = result["populations"][0]
    np.testing.assert_array_equal(pop["spike_ticks"], ref["ticks"])
    np.testing.assert_array_equal(pop["indices"], ref["indices"])
    np.testing.assert_allclose(pop["states"]["v"].astype(np.float64), ref["v"], rtol=1e-4, atol=5e-6)


def test_scaled_cuba_tenth_scale_matches_oracle():
    """Config 3's network at a tenth of its neurons (100k, in-degree 1000, 1e8 synapses, bench weights)."""
    print("case: scaled CUBA 100k x 1000, 150 ticks", flush=True)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=150, weight_scale=0.0116)
    expected = oracle.run(doc, lift_recording_budget=True)
    assert expected.synaptic_events > 1_000_000
    document, result, dump, events = run_gpu(doc, lift_recording_budget=True)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


@pytest.mark.parametrize("full_shape", [False, True])
def test_scaled_cuba_per_edge_weights_tenth_scale_matches_oracle(full_shape):
    """Config 3's network at a tenth of its neurons with a float32 weight per synapse (procedural
    uniform initializers on the device topology, drawn from each row's edge id where read):
    ordered delivery, byte-exact with the oracle over 150 ticks, with the launch shape chosen for
    100k neurons and with the one the full 1M network gets (4096-neuron blocks, several staging
    windows per block and tick)."""
    print(f"case: scaled CUBA 100k x 1000, per-edge weights, 150 ticks, full_shape={full_shape}", flush=True)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=150, weight_scale=0.0116,
                              edge_weights=True)
    expected = oracle.run(doc, lift_recording_budget=True)
    assert expected.synaptic_events > 1_000_000
    shape = engine.choose_shape(1_000_000, 1) if full_shape else None
    with HipExecutor(doc, device=0, lift_recording_budget=True, shape=shape) as ex:
        assert all(path.topology[0] == "fixed_indegree" and set(path.edge_gen) == {"w"}
                   for path in ex.plan.pathways)
        assert not any(engine.counting_group(g) for g in ex.plan.groups)
        result = ex.run()
        dump, events = write_results(ex.document, result), write_events(ex.document, result)
    assert_same_dump(ex.document, dump, expected.results)
    assert events == expected.events


def test_device_topology_matches_oracle():
    """The device Floyd + radix-sort builder writes exactly the oracle's source-major edge list."""
    print("case: device fixed-indegree topology vs oracle", flush=True)
    doc = models.cuba_network(30_000, indegree=150, delay_ticks=1, steps=1)
    with HipExecutor(doc, device=0) as ex:
        for path in ex.plan.pathways:
            _, indegree, seed = path.topology
            src, tgt = oracle.fixed_indegree(path.scount, path.tcount, indegree, seed)
            nb = ex.plan.populations[path.target].blocks
            row_target = ex.sim.read(path.buffers["row_tgt"], np.uint32, path.edge_count)
            seg = ex.sim.read(path.buffers["seg"], np.uint32, path.scount * (nb + 1)).reshape(path.scount, nb + 1)
            np.testing.assert_array_equal(row_target, tgt.astype(np.int64) + path.tstart)
            key = src.astype(np.int64) * nb + (tgt.astype(np.int64) + path.tstart) // ex.plan.shape.block
            first = np.searchsorted(key, np.arange(path.scount * nb).reshape(path.scount, nb))
            np.testing.assert_array_equal(seg[:, :nb], first)
            np.testing.assert_array_equal(seg[:, nb], np.searchsorted(src, np.arange(1, path.scount + 1)))


def check_slots(ex, path, sources):
    """Slot entries of the given sources hold the segment counts and the block-local targets of the
    pathway's row table, in row order, at their XCD-major positions."""
    tpop = ex.plan.populations[path.target]
    nb, block, px = tpop.blocks, ex.plan.shape.block, engine.per_xcd(ex.plan)
    D = len(path.dvals)
    groups = path.scount * D
    longs = 0
    for src in sources:
        for d in range(D):
            g = src * D + d
            seg = ex.sim.read(path.buffers["seg"], np.uint32, nb + 1, offset=g * (nb + 1) * 4)
            for b in range(nb):
                wg = tpop.first_block + b
                y = (wg // px) * groups * px + g * px + wg % px
                slot = ex.sim.read(path.buffers["slot"], np.uint16, 16, offset=y * 32)
                lo, hi = int(seg[b]), int(seg[b + 1])
                assert slot[0] == hi - lo, (src, d, b)
                if hi - lo > engine.SLOT_TARGETS:
                    # a long segment keeps its first row in u32 word 1
                    assert int(slot[2]) | int(slot[3]) << 16 == lo, (src, d, b)
                    longs += 1
                elif hi > lo:
                    rows = ex.sim.read(path.buffers["row_tgt"], np.uint32, hi - lo, offset=lo * 4)
                    assert np.array_equal(slot[1:1 + hi - lo], rows - b * block), (src, d, b)
    return longs


def test_slot_tables_and_their_long_segments():
    """Counting groups deliver through the slot table: segments of up to 15 targets inline, and,
    in a denser projection (in-degree 500 into 256-neuron blocks: ~64 events per segment), longer
    segments through their first row in the slot and the row table.  Both byte-exact with the
    oracle."""
    for n, indegree, dense in ((4000, 50, False), (2000, 500, True)):
        print(f"case: slot tables n={n} indegree={indegree}", flush=True)
        doc = models.cuba_network(n, indegree=indegree, delay_ticks=1, steps=300, weight_scale=0.5)
        expected = oracle.run(doc)
        with HipExecutor(doc, device=0) as ex:
            assert not ex.plan.slot_fallback and "SLOTS = true" in ex.plan.source
            longs = sum(check_slots(ex, path, sources=range(0, path.scount, 7)) for path in ex.plan.pathways)
            assert (longs > 100) == dense
            result = ex.run()
            dump, events = write_results(ex.document, result), write_events(ex.document, result)
        assert_same_dump(ex.document, dump, expected.results)
        assert events == expected.events
        assert expected.synaptic_events > 10_000


def test_full_size_event_conservation():
    """Config 3 at its full size (1M neurons, 1e9 synapses), 60 ticks: every spike emitted before the
    last tick is delivered to exactly its out-degree targets (read from the device rows), and a
    replay reproduces the raster."""
    print("case: scaled CUBA 1M x 1000, 60 ticks, conservation", flush=True)
    doc = models.cuba_network(1_000_000, indegree=1000, delay_ticks=1, steps=60, weight_scale=0.0116)
    with HipExecutor(doc, device=0, lift_recording_budget=True, verify_envelope=False) as ex:
        first = ex.run()
        second = ex.run()
        pop = first["populations"][0]
        assert len(pop["spike_ticks"]) > 10_000
        np.testing.assert_array_equal(pop["indices"], second["populations"][0]["indices"])
        np.testing.assert_array_equal(pop["spike_ticks"], second["populations"][0]["spike_ticks"])
        np.testing.assert_array_equal(pop["states"]["v"], second["populations"][0]["states"]["v"])
        sent = pop["indices"][pop["spike_ticks"] < 59]
        nb = ex.plan.populations[0].blocks
        # pathways run in schedule order (synapses_1_pre sorts before synapses_pre), so each is
        # matched to its own source range and synapse index
        for path in ex.plan.pathways:
            seg = ex.sim.read(path.buffers["seg"], np.uint32, path.scount * (nb + 1)).reshape(path.scount, nb + 1)
            outdeg = seg[:, nb].astype(np.int64) - seg[:, 0]
            assert outdeg.sum() == path.edge_count
            mine = sent[(sent >= path.sstart) & (sent < path.sstart + path.scount)] - path.sstart
            assert first["synapses"][path.synapse]["events"] == int(outdeg[mine].sum())
            # the slot table is complete (counting through it) and agrees with the row table
            assert path.index not in ex.plan.slot_fallback
            check_slots(ex, path, sources=range(0, path.scount, path.scount // 97))
        assert "SLOTS = true" in ex.plan.source


def test_weighted_burst_orders_many_flushes():
    """Distinct per-edge weights force ordered (not counted) delivery; every neuron fires at tick 0,
    so tick 1 stages ~600k events through the LDS buffer in many flushes per block."""
    print("case: per-edge weights, synchronous burst, ordered multi-flush delivery", flush=True)
    doc = nets.weighted_burst()
    expected = oracle.run(doc)
    assert expected.synaptic_events >= 600_000
    with HipExecutor(doc, device=0) as ex:
        assert not any(engine.counting_group(g) for g in ex.plan.groups)
        result = ex.run()
        dump, events = write_results(ex.document, result), write_events(ex.document, result)
    assert_same_dump(ex.document, dump, expected.results)
    assert events == expected.events


def test_runner_cli_writes_the_reference_files(golden, tmp_path):
    """atlas-hip-runner MODEL OUT writes results.bin / events.bin byte-identical to the reference
    b2-runner's, and summary.json with the same counters."""
    print("case: atlas-hip-runner on the reference-v1 fixture", flush=True)
    import json
    from atlas_hip import runner
    out = tmp_path / "out"
    assert runner.main([str(golden / "reference_v1_model.json"), str(out)]) == 0
    assert (out / "results.bin").read_bytes() == (golden / "reference_v1_results.bin").read_bytes()
    assert (out / "events.bin").read_bytes() == (golden / "reference_v1_events.bin").read_bytes()
    mine = json.loads((out / "summary.json").read_text())
    ref = json.loads((golden / "reference_v1_summary.json").read_text())
    for key in ("dump_bytes", "event_dump_bytes", "final_time_seconds", "neuron_count", "population_count",
                "schema", "spike_count", "synaptic_events"):
        assert mine[key] == ref[key], key


def test_device_exponential_bits_equal_the_host():
    """atlas_exp / atlas_expm1 / atlas_exprel evaluated by a gfx950 kernel (hiprtc, same compile
    options as the tick kernels) equal the host build of the same source bit for bit."""
    print("case: device exponential bits, 3 x 1M inputs", flush=True)
    from atlas_hip import native
    n = 1 << 20
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-40, 40, n // 2), rng.uniform(-745, 709.8, n // 4),
                        rng.uniform(-0.006, 0.006, n // 4)])
    source = native.device_header_text().split("typedef unsigned int u32;")[0] + f"""
typedef unsigned long long u64;
typedef long long i64;
extern "C" __global__ void __launch_bounds__(256) math_probe(const u64* __restrict__ tab, i64 tick) {{
    (void)tick;
    const u64 i = (u64)blockIdx.x * 256u + threadIdx.x;
    if (i >= {n}ull) return;
    const double v = reinterpret_cast<const double*>(tab[0])[i];
    reinterpret_cast<double*>(tab[1])[i] = atlas_exp(v);
    reinterpret_cast<double*>(tab[2])[i] = atlas_expm1(v);
    reinterpret_cast<double*>(tab[3])[i] = atlas_exprel(v);
}}
"""
    sim = native.Sim(0)
    try:
        bufs = [sim.alloc(n * 8, x)] + [sim.alloc(n * 8) for _ in range(3)]
        assert bufs == [0, 1, 2, 3]
        sim.compile(source, ["math_probe"], engine.COMPILE_OPTIONS)
        sim.set_schedule([(0, n // 256, 256, 0)])
        sim.run(0, 1)
        for k, fn in enumerate(("exp", "expm1", "exprel"), start=1):
            host, _ = oracle.math(fn, x)
            got = sim.read(k, np.float64, n)
            mismatch = np.flatnonzero(got.view(np.uint64) != host.view(np.uint64))
            assert mismatch.size == 0, (fn, x[mismatch[:5]], got[mismatch[:5]], host[mismatch[:5]])
    finally:
        sim.close()


@pytest.mark.parametrize("dtype", ["f32", "f64"])
def test_hh_ionic_workload_matches_oracle(dtype):
    print(f"case: HH ionic workload {dtype}, 200 x 3000", flush=True)
    doc = nets.hh_ionic_network(200, 3000, dtype=dtype)
    expected = oracle.run(doc, shared_math=True)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


def test_cobahh_matches_oracle():
    """Config 2 (COBAHH, 4000 HH neurons, Bernoulli p = 0.02, delay 0) over its full 10,000 ticks
    (1 s): bit-exact with the oracle in shared-math mode (about a minute of oracle time), which for
    this network equals the libm (reference) mode (test_oracle.py, and the persistent test's libm
    oracle over the same 10,000 ticks)."""
    print("case: COBAHH 4000, 10000 ticks", flush=True)
    doc = models.cobahh_network(4000, steps=10_000)
    expected = oracle.run(doc, shared_math=True)
    assert expected.spike_count > 100_000
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


@pytest.mark.parametrize("neurons,degree,steps", [(64, 8, 400), (2000, 32, 1200)])
def test_stdp_workload_matches_oracle(neurons, degree, steps):
    """On_pre deliveries writing synapse states (ordered), delay-0 and delayed pre events in the
    split kernels, an on_post pathway with a 2-tick delay, event-driven traces with exp."""
    print(f"case: delayed recurrent STDP {neurons}x{degree}, {steps} ticks", flush=True)
    doc = nets.stdp_network(neurons, degree, steps)
    expected = oracle.run(doc, shared_math=True)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    # the host-libm (reference) mode gives the same dump: the trace decays' exp agree after f32 storage
    assert_same_dump(document, dump, oracle.run(doc).results)
    ref = nets.stdp_reference(neurons, degree, steps)
    np.testing.assert_array_equal(result["populations"][0]["spike_ticks"], ref["ticks"])


def test_plastic_network_matches_oracle():
    """Config 5's network at 5000 neurons: STDP on excitatory synapses (ordered on_pre writing
    synapse states, delay-0 on_post), per-edge delays 1-20 ticks, static projections counted."""
    print("case: plastic delayed network 5000 x 1000, 1000 ticks", flush=True)
    doc = models.plastic_network(5000, steps=1000, packed=False)
    expected = oracle.run(doc, shared_math=True, lift_recording_budget=True)
    assert expected.spike_count > 500
    document, result, dump, events = run_gpu(doc, lift_recording_budget=True)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    # the host-libm (reference) mode gives the same dump
    assert_same_dump(document, dump, oracle.run(doc, lift_recording_budget=True).results)


def test_plastic_network_20k_matches_oracle():
    """Config 5's network at 20,000 neurons (2e7 synapses: STDP on 1.28e7 of them, per-edge delays
    1-20), 3000 ticks with about 4e4 spikes and 7e7 synaptic events, through the network's
    synchronous bursts: bit-exact with the oracle (about 90 s of building and oracle time)."""
    print("case: plastic delayed network 20000 x 1000, 3000 ticks", flush=True)
    doc = models.plastic_network(20_000, steps=3000, packed=False)
    expected = oracle.run(doc, shared_math=True, lift_recording_budget=True)
    assert expected.synaptic_events > 50_000_000
    document, result, dump, events = run_gpu(doc, lift_recording_budget=True)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


def test_queued_bursts_and_queue_overflow(monkeypatch):
    """Queued deliveries (ordered group, delays 1-3): synchronous bursts put up to ~20k events
    into one target block in one tick, so the consumer stages them in many windows of whole
    targets, and queues started at 2048 records (no budget for their exact bound) overflow and
    are replayed larger; bit-exact."""
    print("case: queued bursts 1200 x 400, 300 ticks, initial queue 2048", flush=True)
    monkeypatch.setattr(engine, "QUEUE_CAPACITY", 2048)
    monkeypatch.setattr(engine, "QUEUE_BUDGET_BYTES", 0)
    doc = models.plastic_network(1200, indegree=400, delays=(1, 3), steps=300, we=5e-3, wmax=2e-2, packed=False)
    expected = oracle.run(doc, shared_math=True, lift_recording_budget=True)
    with HipExecutor(doc, device=0, lift_recording_budget=True) as ex:
        assert ex.plan.queues, "the plastic group should be queued"
        result = ex.run()
        assert max(q["cap"] for q in ex.plan.queues.values()) > 2048
        dump, events = write_results(ex.document, result), write_events(ex.document, result)
        document = ex.document
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


@pytest.mark.parametrize("delay", [0, 1])
def test_poisson_group_matches_oracle(delay):
    """A PoissonGroup (threshold rand() < rates * dt on the counter RNG, per-neuron rates) driving
    CUBA neurons: the device draws counter_uniform(seed, stream, tick, neuron) bit for bit, so
    the Poisson raster, the driven raster and every state equal the oracle's."""
    print(f"case: poisson group 2000 -> 4000, delay {delay}, 2000 ticks", flush=True)
    doc = models.poisson_network(2000, 4000, steps=2000, delay_ticks=delay)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    poisson, driven = (len(p["spike_ticks"]) for p in result["populations"])
    assert poisson > 5000 and driven > 1000


@pytest.mark.parametrize("variant", ["rand", "randn", "procedural", "cuba-delay0", "cuba-delay1"])
def test_random_pathway_draws_match_oracle(variant):
    """Pathway programs drawing from the counter RNG per event (rand() and randn() indexed by the
    edge, at the delivery tick): an f64 accumulator driven by a spike generator through a shuffled
    explicit topology (each row reads its edge index from a table) or a procedural one (rows in edge
    order), and CUBA neurons with ge += w (0.5 + rand()) at delay 0 and 1; every state and raster
    equals the oracle's (in shared-math mode: randn's logarithm is the shared correctly rounded
    one, which the host libm may miss by an ulp)."""
    print(f"case: random pathway draws, {variant}", flush=True)
    kwargs = {"rand": {}, "randn": {"draw": "randn"}, "procedural": {"procedural": True},
              "cuba-delay0": {"cuba": True, "delay_ticks": 0, "n": 1000, "steps": 2000},
              "cuba-delay1": {"cuba": True, "delay_ticks": 1, "n": 1000, "steps": 2000}}[variant]
    doc = models.random_pathway_network(**kwargs)
    expected = oracle.run(doc, shared_math=True)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    if kwargs.get("cuba"):
        assert len(result["populations"][1]["spike_ticks"]) > 500


@pytest.mark.parametrize("case", ["reference", "reference-1000", "custom-only", "custom-only-unrecorded",
                                  "cuba-delay1", "cuba-delay0"])
def test_custom_events_match_oracle(case):
    """Named events beside the spike: conditions at the threshold, run_on_event code in the resets
    slot in schedule order, EventMonitors at the threshold and at the end of the tick, every event's
    stream: the reference test's network (4 neurons, and 1000 of them over 1000 ticks), a
    custom-only population, and CUBA neurons with a custom event and spike-triggered deliveries at
    delay 1 and 0.  results.bin and events.bin equal the oracle's."""
    print(f"case: custom events, {case}", flush=True)
    doc = {"reference": lambda: nets.custom_event_network(),
           "reference-1000": lambda: nets.custom_event_network(scale=250, steps=1000),
           "custom-only": lambda: nets.custom_only_network(),
           "custom-only-unrecorded": lambda: nets.custom_only_network(record=False),
           "cuba-delay1": lambda: nets.custom_cuba_network(delay_ticks=1),
           "cuba-delay0": lambda: nets.custom_cuba_network(delay_ticks=0)}[case]()
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


@pytest.mark.parametrize("case", ["reference", "reference-delay1", "one-clock", "one-clock-delay2",
                                  "reference-mutable", "one-clock-mutable-delay1", "one-clock-post0",
                                  "one-clock-post2", "one-clock-post-per-edge", "one-clock-post-per-edge-delay1",
                                  "reference-mutable-post",
                                  "cuba-routes", "cuba-routes-delay0", "cuba-routes-shared"])
def test_custom_event_routes_match_oracle(case):
    """Pathways triggered by custom events, several on_pre pathways per Synapses: the reference's
    route test network (spike, alpha and zeta pathways into a target on a clock of 2 dt, delays
    0-3 ticks; with every delay one tick longer; on one clock; with w a synapse state all three
    pathways raise; with an on_post pathway on the target's reply event, one delay or per-edge
    delays, on one clock or the target's own: the reference test's mutable case), and CUBA neurons whose high event and spike drive a recurrent Synapses
    (per-edge delays 1-3 or 0-2 ticks; both pathways updating one synapse state).  results.bin and
    events.bin equal the oracle's."""
    print(f"case: custom event routes, {case}", flush=True)
    doc = {"reference": lambda: nets.custom_route_network(),
           "reference-delay1": lambda: nets.custom_route_network(delay_shift=1),
           "one-clock": lambda: nets.custom_route_network(two_clocks=False),
           "one-clock-delay2": lambda: nets.custom_route_network(delay_shift=2, two_clocks=False),
           "reference-mutable": lambda: nets.custom_route_network(mutable=True),
           "one-clock-mutable-delay1": lambda: nets.custom_route_network(delay_shift=1, two_clocks=False,
                                                                        mutable=True),
           "one-clock-post0": lambda: nets.custom_route_network(two_clocks=False, mutable=True, post_delay=0),
           "one-clock-post2": lambda: nets.custom_route_network(delay_shift=1, two_clocks=False, mutable=True,
                                                               post_delay=2),
           "one-clock-post-per-edge": lambda: nets.custom_route_network(two_clocks=False, mutable=True,
                                                                       post_delay=[0, 1, 2, 1, 3]),
           "one-clock-post-per-edge-delay1": lambda: nets.custom_route_network(
               delay_shift=1, two_clocks=False, mutable=True, post_delay=[2, 0, 1, 3, 1]),
           "reference-mutable-post": lambda: nets.custom_route_network(mutable=True, post_delay=[0, 1, 2, 1, 3]),
           "cuba-routes-shared": lambda: nets.custom_cuba_network(2000, steps=2000, routes=(1, 3), counted=True),
           "cuba-routes": lambda: nets.custom_cuba_network(2000, steps=2000, routes=(1, 3)),
           "cuba-routes-delay0": lambda: nets.custom_cuba_network(2000, steps=2000, routes=(0, 2))}[case]()
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    assert expected.synaptic_events > 0


def test_vector_log_matches_oracle():
    """log() in vector code through the shared correctly rounded atlas_log (the oracle in shared-math
    mode evaluates the same function; the host libm may differ by an ulp on rare arguments): states
    and the raster of neurons driven by logarithms of random draws equal the oracle's."""
    print("case: vector log, 2000 neurons, 1000 ticks", flush=True)
    doc = nets.log_network(2000, steps=1000)
    expected = oracle.run(doc, shared_math=True)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert expected.spike_count > 1000


@pytest.mark.parametrize("threshold", [False, True])
def test_scalar_draws_match_oracle(threshold):
    """A scalar statement drawing rand() once per tick (index 0, shared by every neuron) and a vector
    statement drawing per neuron, with and without a threshold on the result: states and raster
    equal the oracle's."""
    print(f"case: scalar draws, threshold={threshold}", flush=True)
    doc = nets.shared_draw_network(4000, steps=2000, threshold=threshold)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    if threshold:
        assert expected.spike_count > 10_000


@pytest.mark.parametrize("delay", [0, 2])
def test_spike_generator_matches_oracle(delay):
    """A SpikeGeneratorGroup (20k scheduled spikes and a synchronous volley of all 500 inputs at
    tick 10) driving CUBA neurons: each generator neuron fires when its next scheduled tick comes
    up; the generator raster equals its schedule and the run equals the oracle's."""
    print(f"case: spike generator 500 -> 1000, delay {delay}, 2000 ticks", flush=True)
    doc = models.generator_network(delay_ticks=delay)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    schedule = doc["instance"]["populations"][0]["spike_generator"]
    np.testing.assert_array_equal(result["populations"][0]["spike_ticks"], schedule["spike_ticks"])
    np.testing.assert_array_equal(result["populations"][0]["indices"], schedule["spike_indices"])


@pytest.mark.parametrize("delay", [0, 1])
def test_event_monitor_matches_oracle(delay):
    """An EventMonitor recording v, ge (states) and Vt (a scalar parameter) at each spike, at the
    threshold before the reset: the device appends records as neurons fire and the host orders
    them by (tick, neuron); events.bin, with its monitor section, equals the oracle's."""
    print(f"case: event monitor CUBA 4000, delay {delay}, 1000 ticks", flush=True)
    kwargs = dict(delay_ticks=1, indegree=100, weight_scale=0.5) if delay else {}
    doc = models.cuba_network(4000, steps=1000, event_monitor=["v", "ge", "Vt"], **kwargs)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    monitor = result["populations"][0]["event_monitors"]["neurongroup_eventmonitor"]
    assert len(monitor["ticks"]) == len(result["populations"][0]["spike_ticks"]) > 100


@pytest.mark.parametrize("model,boundary", [("fixture", 128), ("cuba_delay3", 200), ("cuba_indegree", 150),
                                            ("plastic", 705), ("stdp", 200), ("routes", 5), ("routes_clocks", 6),
                                            ("multiclock", 300), ("routes_restore", 4)])
def test_continuation_equals_the_continuous_run(golden, model, boundary):
    """A run split in two on the GPU, the second segment built from the first one's results
    (final states, refractory and synapse states, pending delayed events), equals the oracle
    on the same continuation document and ends bit-identical to the continuous run; also for the
    reference route test's network, on one clock and on its two (pending events of pathways on
    custom events and of its on_post pathway on the target's reply event, each counted in the
    ticks of its own clock; split after 4 ticks with the on_post pathway's per-edge delays, as the
    reference's segment test test_gpu_custom_events.py:76-100 does), and three CUBA populations on
    three clocks."""
    import json
    from atlas_hip import protocol
    from atlas_hip.continuation import continuation, first_segment
    document = {"fixture": lambda: json.loads((golden / "reference_v1_model.json").read_text()),
                "cuba_delay3": lambda: models.cuba_network(1000, steps=400, delay_ticks=3),
                "cuba_indegree": lambda: models.cuba_network(5000, indegree=100, delay_ticks=3, weight_scale=0.35,
                                                             steps=300),
                "plastic": lambda: models.plastic_network(2000, steps=1000, packed=False),
                "stdp": lambda: nets.stdp_network(64, 8, 400),
                "routes": lambda: nets.custom_route_network(two_clocks=False, mutable=True, post_delay=2,
                                                            delay_shift=1),
                "routes_clocks": lambda: nets.custom_route_network(mutable=True, post_delay=1, delay_shift=1),
                "multiclock": lambda: nets.multiclock_network(3000, steps=600, monitor=False),
                "routes_restore": lambda: nets.custom_route_network(mutable=True, post_delay=[0, 1, 2, 1, 3])}[model]()
    steps = protocol.load(document)["run"]["clocks"][0]["steps"]
    print(f"continuation {model} at {boundary}", flush=True)
    _, full, full_dump, _ = run_gpu(document, lift_recording_budget=True)
    first_doc = first_segment(document, boundary)
    _, first, _, _ = run_gpu(first_doc, lift_recording_budget=True)
    second_doc = continuation(first_doc, first, steps - boundary)
    assert sum(len(pw["pending"]) for s in second_doc["instance"]["synapses"] for pw in s["pathways"]) > 0
    doc2, second, dump2, _ = run_gpu(second_doc, lift_recording_budget=True)
    assert_same_dump(doc2, dump2, oracle.run(second_doc, shared_math=True, lift_recording_budget=True).results)
    a, b = read_results(full_dump, protocol.load(document)), read_results(dump2, doc2)
    d = protocol.load(document)["definition"]
    dt = [struct.unpack(">d", bytes.fromhex(c["dt"]))[0] for c in d["clocks"]]
    d2 = protocol.load(doc2)["definition"]
    for pa, pb, pdef, pdef2 in zip(a.populations, b.populations, d["populations"], d2["populations"]):
        mine = int(round(boundary * dt[0] / dt[pdef["clock"]]))   # the boundary in the population's ticks
        # the second segment records its last window_steps ticks
        recorded = mine + int(pdef2["steps"]) - int(pdef2["monitor"]["window_steps"])
        assert np.array_equal(pa.spikes[pa.spikes[:, 0] >= recorded], pb.spikes)
        for x, y in zip(pa.states, pb.states):
            assert np.array_equal(np.asarray(x).view(np.uint8), np.asarray(y).view(np.uint8))
    for sa, sb in zip(full["synapses"], second["synapses"]):
        for name in sa["states"]:
            assert np.array_equal(sa["states"][name].view(np.uint8), sb["states"][name].view(np.uint8))
    assert [f["events"] + s["events"] for f, s in zip(first["synapses"], second["synapses"])] == \
        [s["events"] for s in full["synapses"]]


@pytest.mark.parametrize("model", ["reference_example", "weighted_cuba"])
def test_binary_csr_topology_matches_oracle(tmp_path, model):
    """Edges from a B2CSR001 file (the reference's conformance model, and CUBA with per-edge
    weights: an ordered on_pre) give the dump the oracle gives for the same edges inline."""
    doc = models.binary_csr_example()[0] if model == "reference_example" else nets.weighted_cuba()
    binary = models.to_binary_csr(doc, 0, tmp_path / "graph.b2csr")
    print(f"binary csr {model}", flush=True)
    document, _, dump, _ = run_gpu(binary)
    assert_same_dump(document, dump, oracle.run(doc, shared_math=True).results)


@pytest.mark.parametrize("delay", [0, 1])
def test_poisson_input_network_matches_oracle(delay):
    """CUBA neurons driven by two PoissonInputs (ge: N = 1000 at 500 Hz, the normal
    approximation; gi: N = 50 at 20 Hz, inversion), recurrent delays 0 and 1: bit-exact."""
    doc = models.cuba_network(1000, steps=300, delay_ticks=delay,
                              poisson_inputs=(("ge", 1000, 500.0, 0.02e-3), ("gi", 50, 20.0, -0.1e-3)))
    print(f"poisson input delay {delay}", flush=True)
    document, _, dump, _ = run_gpu(doc)
    assert_same_dump(document, dump, oracle.run(doc, shared_math=True).results)


@pytest.mark.parametrize("count,rate", [(20, 100.0), (1000, 500.0), (3, 9000.0)])
def test_poisson_input_draws_match_oracle(count, rate):
    """Accumulated PoissonInput draws of 20,000 neurons over 40 ticks, bit for bit: inversion
    (N p = 0.2), the normal approximation (N p = 50) and the reversed tail (p = 0.9 > 0.5)."""
    builder = models.NetworkBuilder(dt=1e-4, steps=40, seed=99)
    pop = builder.population("inputs", 20000, states={"x": ("f64", models.DIMLESS, np.zeros(20000))},
                             spike_monitor=False)
    builder.poisson_input(pop, "x", count, rate, 1.0)
    doc = builder.document()
    print(f"poisson input draws N={count} rate={rate}", flush=True)
    document, _, dump, _ = run_gpu(doc)
    assert_same_dump(document, dump, oracle.run(doc, shared_math=True).results)


def test_noisy_lif_matches_oracle():
    """White-noise LIF (randn() in the update, Euler-Maruyama): spikes and states bit-exact."""
    doc = nets.noisy_lif()
    print("noisy lif", flush=True)
    document, _, dump, _ = run_gpu(doc)
    assert_same_dump(document, dump, oracle.run(doc, shared_math=True).results)


@pytest.mark.parametrize("lam", [3.0, 50.0])
def test_poisson_draws_match_oracle(lam):
    """poisson() in neuron code (the product method and PTRS): accumulated draws of 20,000
    neurons over 40 ticks, bit for bit."""
    builder = models.NetworkBuilder(dt=1e-4, steps=40, seed=5)
    draw = {"op": "poisson", "stream": 4, "lambda": models.ld("lam")}
    builder.population("x", 20000, states={"x": ("f64", models.DIMLESS, np.zeros(20000))},
                       parameters={"lam": ("f64", models.DIMLESS, lam)},
                       update=([], [models.stmt("x", "f64", models.add(models.ld("x"), draw))]), spike_monitor=False)
    doc = builder.document()
    print(f"poisson draws lambda={lam}", flush=True)
    document, _, dump, _ = run_gpu(doc)
    assert_same_dump(document, dump, oracle.run(doc, shared_math=True).results)


def test_executor_result_satisfies_the_reference_writer(golden, tmp_path):
    """HipExecutor.run() through the reference result writer (metal.py:926-1014, restated in
    tests/reference_writer.py), as the INTEGRATION binding calls it: it runs to completion and
    writes the golden dump; a model with random draws reports the CPU engine's counter profile,
    which the binding's one-line change accepts."""
    import reference_writer
    print("case: executor result contract", flush=True)
    with HipExecutor(golden / "reference_v1_model.json", device=0) as ex:
        result = ex.run()
        document = ex.document
    assert result["rng_profile"] is None
    assert [set(t) for t in result["timings"]] == [{"input_seconds", "command_seconds", "gpu_seconds",
                                                    "readback_seconds"}]
    assert "gfx950" in result["device"]
    summary = reference_writer.write_gpu_results(document, result, tmp_path / "fixture", engine="hip",
                                                 numeric_profile=result["numeric_profile"])
    assert (tmp_path / "fixture" / "results.bin").read_bytes() == (golden / "reference_v1_results.bin").read_bytes()
    assert (tmp_path / "fixture" / "events.bin").read_bytes() == (golden / "reference_v1_events.bin").read_bytes()
    assert summary["spike_count"] == 155 and summary["synaptic_events"] == 1238
    doc = models.poisson_network(200, 300, indegree=20, steps=50)
    with HipExecutor(doc, device=0) as ex:
        result = ex.run()
        document = ex.document
    assert result["rng_profile"] == document["definition"]["rng_algorithm"] == "splitmix64-counter-v1"
    with pytest.raises(reference_writer.ConsumerRejected):
        reference_writer.write_gpu_results(document, result, tmp_path / "strict", engine="hip",
                                           numeric_profile=result["numeric_profile"])
    reference_writer.write_gpu_results(document, result, tmp_path / "random", engine="hip",
                                       numeric_profile=result["numeric_profile"],
                                       rng_profile=document["definition"]["rng_algorithm"])
    assert (tmp_path / "random" / "results.bin").read_bytes() == write_results(document, result)


@pytest.mark.parametrize("kind", ["overflow", "clip", "divisor", "exp", "events"])
def test_nonfinite_values_fail_at_the_oracle_tick(kind):
    """The finiteness checks the engine keeps fail the run at exactly the tick count where the
    oracle's per-operation checks do, and the run one tick shorter equals the oracle's."""
    print(f"case: non-finite {kind}", flush=True)
    first = None
    for steps in range(1, 9):
        try:
            oracle.run(nets.nonfinite_network(kind, steps))
        except oracle.OracleError as error:
            assert "non-finite" in str(error)
            first = steps
            break
    assert first is not None and first >= 2
    expected = oracle.run(nets.nonfinite_network(kind, first - 1))
    document, _, dump, _ = run_gpu(nets.nonfinite_network(kind, first - 1))
    assert_same_dump(document, dump, expected.results)
    with pytest.raises(FloatingPointError, match="non-finite"):
        run_gpu(nets.nonfinite_network(kind, first))


@pytest.mark.parametrize("kind,distribution", [("total", "uniform"), ("total", "normal"), ("indegree", "uniform"),
                                               ("indegree", "normal")])
def test_procedural_initialization_equals_the_reference_test(kind, distribution):
    """The model of test_gpu_initialization.py:63-101 on the GPU: fixed-total or fixed-in-degree
    edges, per-edge weight and delay initializers (uniform or clipped normal), delays quantised as
    floor(delay/dt + 0.5), delivery in (delay descending, source, edge) order.  Byte-exact with the
    oracle, and the target's v and trace equal the reference test's own expectation."""
    print(f"case: procedural initialization {kind} {distribution}", flush=True)
    doc = nets.initialization_network(kind, distribution)
    expected = oracle.run(doc)
    document, _, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    target = read_results(dump, document).populations[1]
    reference = nets.initialization_expected(kind, distribution)
    assert np.array_equal(target.states[0], reference["v"])
    assert np.array_equal(target.samples[0], reference["trace"])
    assert expected.synaptic_events == reference["events"]


def test_procedural_cuba_100k_matches_oracle():
    """100k CUBA neurons whose projections the engine draws itself: fixed in-degree with uniform
    per-edge weights and fixed total (with replacement) with clipped-normal weights, both with
    uniform delay initializers over 1..20 ticks (ordered, queued delivery), 300 ticks."""
    print("case: procedural CUBA 100k x 100 with initializers, 300 ticks", flush=True)
    doc = nets.procedural_cuba(100_000, steps=300)
    expected = oracle.run(doc)
    assert expected.synaptic_events > 1_000_000
    document, _, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


@pytest.mark.parametrize("case", ["order_f32", "reverse_f32", "order_f64", "range", "decay", "dyadic"])
def test_summed_variable_pins_match_oracle(case):
    """The oracle's closed-form pin networks for summed variables and clock-driven synapse
    states on the GPU: edge-order f32 rounding, the endpoint range's zero fill, decay and order
    within the groups slot, exact dyadic sums to both endpoints."""
    print(f"case: summed pin {case}", flush=True)
    tiny = 2.0**-24
    rng = np.random.default_rng(5)
    doc = {
        "order_f32": lambda: nets.summed_pin_network([0, 1, 2], [3, 3, 3], [1.0, tiny, tiny]),
        "reverse_f32": lambda: nets.summed_pin_network([0, 1, 2], [3, 3, 3], [tiny, tiny, 1.0]),
        "order_f64": lambda: nets.summed_pin_network([0, 1, 2], [3, 3, 3], [1.0, tiny, tiny], dtype="f64"),
        "range": lambda: nets.summed_pin_network([0, 1], [1, 1], [0.25, 0.5], target_range=(2, 4)),
        "decay": lambda: nets.summed_pin_network([0, 2], [1, 1], [1.0, 3.0], decay=0.5, steps=10),
        "dyadic": lambda: nets.summed_pin_network(rng.integers(0, 16, 60), rng.integers(0, 16, 60),
                                                  rng.integers(0, 1024, 60) / 256.0, n=16, scale=2.0),
    }[case]()
    expected = oracle.run(doc)
    document, _, dump, events = run_gpu(doc)
    assert dump == expected.results and events == expected.events


@pytest.mark.parametrize("dtype,delay", [("f32", 1), ("f64", 1), ("f32", 3), ("f32", 0), ("f64", 0)])
def test_summed_network_matches_oracle(dtype, delay):
    """10k LIF neurons whose current is the summed variable g (E - v_post) of 5e5 synapses with
    a clock-driven decaying g (plus a summed variable to the sources), 200 ticks: raster, neuron
    and synapse states byte-exact with the oracle.  At delay 0 the synapse programs run between the
    previous tick's deliveries and the update, in launches of their own."""
    print(f"case: summed network 10k x 50 {dtype} delay {delay}", flush=True)
    doc = nets.summed_network(10_000, indegree=50, steps=200, dtype=dtype, delay_ticks=delay)
    expected = oracle.run(doc)
    assert expected.synaptic_events > 100_000
    document, _, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert dump == expected.results and events == expected.events


def test_summed_multiclock_network_matches_oracle():
    """Summed variables and a clock-driven synapse state across two clocks: g decays on the source's
    clock (0.1 ms), the summed current into the targets runs on their clock (0.2 ms) and the
    summed J into the sources on theirs; each runs in the merged steps its clock advances, at its
    own tick and time.  Rasters and all states byte-exact with the oracle."""
    print("case: summed variables across clocks, 4000 + 4000, 600 ticks", flush=True)
    doc = nets.summed_multiclock_network(4000, steps=600)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert all(len(p["spike_ticks"]) > 5000 for p in result["populations"])


@pytest.mark.parametrize("n,steps,per_edge,zero", [(3000, 600, False, False), (3000, 600, True, False),
                                                    (30_000, 1200, False, False), (3000, 600, False, True),
                                                    (3000, 600, True, True)])
def test_multiclock_network_matches_oracle(n, steps, per_edge, zero):
    """Three populations on clocks of dt, 1.5 dt and 2 dt coupled in a ring (pushed counts with
    delays of 1-3 ticks, counted pulls, and, with ``per_edge``, ordered deliveries of per-edge
    weights), one launch per merged step: rasters, monitored traces, states and delivered counts
    byte-exact with the oracle.  With ``zero`` two of the pathways have delay-0 events, and each
    merged step is two launches: the updates, then the deliveries, on_post pathways and resets."""
    print(f"case: multiclock {n} x {steps} per_edge={per_edge} zero_delay={zero}", flush=True)
    doc = nets.multiclock_network(n, steps=steps, per_edge=per_edge, zero_delay=zero)
    expected = oracle.run(doc)
    assert expected.synaptic_events > 100_000
    document, _, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert dump == expected.results and events == expected.events


@pytest.mark.parametrize("source_clock,delay,ticks", [(1, 2, [0, 5, 37, 38]), (0, 3, [0, 10, 56, 57])])
def test_multiclock_arrivals_match_oracle(source_clock, delay, ticks):
    """A generator on one clock into an accumulator on another (coincident ticks, arrivals after
    the target's last tick, one beyond the source's run): the monitored trace and final state
    byte-exact with the oracle, whose arrival times are pinned in closed form."""
    print(f"case: clock arrivals source clock {source_clock} delay {delay}", flush=True)
    doc = nets.clock_arrival_network(source_clock, delay, ticks, [0, 1, 0, 1])
    expected = oracle.run(doc)
    document, _, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert dump == expected.results and events == expected.events


def test_plastic_network_full_size_conservation_and_replay():
    """Config 5 at its own size (100k neurons, in-degree 1000, 1e8 synapses, delays 1-20, STDP on
    the 6.4e7 excitatory synapses), 300 ticks: the queued group's records are sized at their exact
    bound, so the run never overflows or replays; every synapse's delivered events equal those
    the raster and the topology imply (each spike's out-edges whose arrival tick lies inside the
    run, plus each target spike's in-edges for the on_post pathway of delay 0); a second run of
    the same executor gives the same dump byte for byte."""
    print("case: plastic 100k x 1000, 300 ticks (conservation, replay)", flush=True)
    steps = 300
    doc = models.plastic_network(100_000, steps=steps)
    inst = doc["instance"]
    with HipExecutor(doc, device=0, lift_recording_budget=True, verify_envelope=False) as ex:
        queued = {k: dict(v) for k, v in ex.plan.queues.items()}
        assert queued and all(q["cap"] == q["limit"] for q in queued.values())
        first = ex.run()
        assert ex.plan.queues == queued, "the queues grew: the run was replayed"
        dump = write_results(ex.document, first)
        second = ex.run()
        assert write_results(ex.document, second) == dump
        document = ex.document
    ticks = np.asarray(first["populations"][0]["spike_ticks"], np.int64)
    ids = np.asarray(first["populations"][0]["indices"], np.int64)
    assert ticks.size > 1000
    for k, (sdef, sin) in enumerate(zip(document["definition"]["synapses"], inst["synapses"])):
        src = np.asarray(sin["source"], np.int64)
        tgt = np.asarray(sin["target"], np.int64)
        delay = np.asarray(sin["pathways"][0]["delay_ticks"], np.int64)
        # out-edges per (source, delay), summed over delays below each bound
        deg = np.bincount(src * 22 + delay, minlength=sdef["source_count"] * 22).reshape(-1, 22)
        cum = np.concatenate([np.zeros((deg.shape[0], 1), np.int64), np.cumsum(deg, axis=1)], axis=1)
        mine = (ids >= sdef["source_start"]) & (ids < sdef["source_start"] + sdef["source_count"])
        room = np.minimum(steps - ticks[mine], 22)
        expected = int(cum[ids[mine] - sdef["source_start"], room].sum())
        if len(sin["pathways"]) == 2:
            indegree = np.bincount(tgt, minlength=sdef["target_count"])
            post = (ids >= sdef["target_start"]) & (ids < sdef["target_start"] + sdef["target_count"])
            expected += int(indegree[ids[post] - sdef["target_start"]].sum())
        assert first["synapses"][k]["events"] == expected, (k, first["synapses"][k]["events"], expected)


def test_recording_window_bounds_monitors_across_runs():
    """The reference's recording-window test (test_device.py:554-577) on the device: a 5-tick run
    with a 3-tick window records ticks 2, 3, 4 (count 3), the continuation's 5 ticks record 7, 8,
    9 (count 3); both dumps byte-exact with the oracle."""
    from atlas_hip.continuation import continuation
    print("case: recording window, one neuron, 5 + 5 ticks", flush=True)
    doc = nets.window_neuron(5)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert dump == expected.results and events == expected.events
    assert read_results(dump, document).populations[0].spikes[:, 0].tolist() == [2, 3, 4]
    following = continuation(document, result, 5)
    expected = oracle.run(following)
    document, result, dump, events = run_gpu(following)
    assert dump == expected.results and events == expected.events
    pop = read_results(dump, document).populations[0]
    assert pop.spikes[:, 0].tolist() == [7, 8, 9] and pop.counts.tolist() == [3]


def test_recording_window_shorter_than_the_run_matches_oracle():
    """CUBA 4000 over 2000 ticks with a 700-tick window over v and ge of 40 neurons (state
    samples, spike raster, counts and the event stream of the last 700 ticks), then a
    continuation of 1000 ticks with the same window: byte-exact with the oracle."""
    from atlas_hip.continuation import continuation
    print("case: recording window 700 of CUBA 4000 x 2000, continuation 1000", flush=True)
    doc = models.with_recording_window(
        models.cuba_network(4000, steps=2000, state_monitor=(["v", "ge"], list(range(0, 4000, 100)))), 700)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events
    pop = read_results(dump, document).populations[0]
    assert pop.samples[0].shape == (700, 40) and pop.spikes[:, 0].min() >= 1300
    following = continuation(document, result, 1000)
    expected = oracle.run(following)
    document, result, dump, events = run_gpu(following)
    assert_same_dump(document, dump, expected.results)
    assert events == expected.events


def test_recording_window_in_a_persistent_launch(monkeypatch):
    """Config 3's network at 100k x 1000 (delay 1) over 150 ticks with a 60-tick window: the
    persistent launch writes the recording bitmap from tick 90 on; equal to the oracle."""
    print("case: recording window 60 of persistent CUBA 100k x 1000, 150 ticks", flush=True)
    monkeypatch.setenv("ATLAS_HIP_PERSISTENT", "1")
    doc = models.with_recording_window(
        models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=150, weight_scale=0.0116), 60)
    expected = oracle.run(doc, lift_recording_budget=True)
    with HipExecutor(doc, device=0, lift_recording_budget=True) as ex:
        result = ex.run()
        assert result["hip_runtime"]["launch_mode"] == "persistent"
        dump, events = write_results(ex.document, result), write_events(ex.document, result)
    assert dump == expected.results and events == expected.events


@pytest.mark.parametrize("counter_when", ["start", "end"])
def test_run_regularly_counter_matches_oracle(counter_when):
    """run_regularly code before the update, between the update and the threshold, and at the end of
    the tick (executor.rs:4139-4148), on three f64 counters: byte-exact with the oracle, whose
    closed forms test_oracle.py pins."""
    print(f"case: run_regularly counters, counter at {counter_when}", flush=True)
    doc = nets.regular_counter(50, counter_when=counter_when)
    expected = oracle.run(doc)
    document, result, dump, events = run_gpu(doc)
    assert dump == expected.results and events == expected.events


@pytest.mark.parametrize("end,delay", [(True, 1), (False, 1), (True, 0)])
def test_run_regularly_cuba_matches_oracle(end, delay, monkeypatch):
    """CUBA 4000 with run_regularly code at the start of the tick (gi decayed), after the update (v
    nudged) and, with `end`, after the reset (ge driven), 2000 ticks: bit-exact with the oracle.
    Without the end-of-tick code the plan runs persistent (the code inside the update).  At delay 0
    the end code runs with the previous tick's deliveries and resets, in the launch before the
    update."""
    print(f"case: run_regularly CUBA 4000, end={end}, delay {delay}", flush=True)
    monkeypatch.setenv("ATLAS_HIP_PERSISTENT", "1")
    doc = nets.regular_cuba(4000, 2000, end=end, delay_ticks=delay)
    expected = oracle.run(doc)
    with HipExecutor(doc, device=0) as ex:
        result = ex.run()
        assert result["hip_runtime"]["launch_mode"] == ("per-tick" if end else "persistent")
        dump, events = write_results(ex.document, result), write_events(ex.document, result)
    assert_same_dump(ex.document, dump, expected.results)
    assert events == expected.events
    assert expected.spike_count > 1000
