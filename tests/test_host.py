"""Host side of the HIP engine without a GPU: lowering, layouts, refractory
deadlines, code generation (hiprtc compile for gfx950) and model rejection."""
import copy
import json
import math

import numpy as np
import pytest

import nets
from atlas_hip import engine, models, native, protocol, rtc
from oracle import oracle


def _generate(document):
    plan = engine.lower(document)
    engine.allocate(plan)
    engine.generate(plan, native.device_header_text())
    return plan


@pytest.fixture(scope="module")
def fixture_doc(golden):
    return json.loads((golden / "reference_v1_model.json").read_text())


@pytest.mark.parametrize("name", ["fixture", "cuba_bernoulli", "cuba_indegree_delay3", "delta_lif", "chronology",
                                  "readme", "recurrent", "stdp", "cobahh", "poisson", "generator",
                                  "event_monitor", "poisson_input", "multiclock"])
def test_generated_module_compiles_for_gfx950(name, fixture_doc):
    document = {
        "fixture": lambda: fixture_doc,
        "cuba_bernoulli": lambda: models.cuba_network(1000, steps=50),
        "cuba_indegree_delay3": lambda: models.cuba_network(5000, indegree=100, delay_ticks=3, steps=50),
        "delta_lif": lambda: models.delta_lif_network(3000, indegree=50, steps=50),
        "chronology": nets.chronology_kat,
        "readme": nets.readme_lif,
        "recurrent": lambda: nets.recurrent_network(200, 20, 50),
        "stdp": lambda: nets.stdp_network(64, 8, 20),
        "cobahh": lambda: models.cobahh_network(500, steps=20),
        "poisson": lambda: models.poisson_network(300, 500, indegree=20, steps=20),
        "generator": lambda: models.generator_network(200, 300, spikes=500, indegree=20, steps=50),
        "event_monitor": lambda: models.cuba_network(1000, steps=50, event_monitor=["v", "ge", "Vt"]),
        "poisson_input": lambda: models.cuba_network(1000, steps=50, poisson_inputs=(("ge", 1000, 500.0, 2e-5),)),
        "multiclock": lambda: nets.multiclock_network(600, steps=60),
    }[name]()
    plan = _generate(document)
    code = rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)
    assert len(code) > 1000
    for kernel in plan.kernels:
        assert f'extern "C" __global__' in plan.source and kernel in plan.source
    # every launch covers every 1024-neuron block, padded to whole XCD rounds
    for _, grid, threads, _ in plan.launches:
        assert threads == plan.shape.wg and grid % engine.XCDS == 0 and grid >= plan.total_blocks


def test_row_table_fallback_of_a_counting_group_compiles():
    """A counting group whose slot table overflowed is generated on the row-table delivery."""
    plan = _generate(models.cuba_network(1000, steps=50))
    assert "SLOTS = true" in plan.source and plan.pathways[0].buffers.get("slot") is not None
    plan.slot_fallback.update(path.index for path in plan.pathways)
    engine.generate(plan, native.device_header_text())
    assert "SLOTS = true" not in plan.source and "SLOTS = false" in plan.source
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000


def test_push_and_queued_groups_of_the_plastic_network(monkeypatch):
    """Several delays: the counting group is pushed (arrival counters, no slot tables) and the
    ordered STDP group queued, with queues sized at their exact bound (in-edges per target
    block) when that fits the queue budget, and at the initial capacity under it otherwise; a
    target with more in-edges than one staging window keeps the ordered group on the pull."""
    plan = _generate(models.plastic_network(3000, steps=20, packed=False))
    counting = [g for g in plan.groups if engine.counting_group(g)]
    ordered = [g for g in plan.groups if not engine.counting_group(g)]
    assert counting and ordered
    assert all(engine.push_group(plan, g) and "arrivals" in g[0].buffers for g in counting)
    assert not any("slot" in path.buffers for g in counting for path in g)
    info = plan.queues[ordered[0][0].index]
    assert info == dict(limit=256 * 800, cap=256 * 800, depth=21)
    monkeypatch.setattr(engine, "QUEUE_BUDGET_BYTES", 0)
    small = _generate(models.plastic_network(3000, steps=20, packed=False))
    assert small.queues[ordered[0][0].index] == dict(limit=256 * 800, cap=engine.QUEUE_CAPACITY, depth=21)
    assert "QUEUE = true" in plan.source and "push_events<" in plan.source and "take_events<" in plan.source
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000
    dense = _generate(models.plastic_network(3000, indegree=1500, steps=20, packed=False))
    assert not dense.queues and "take_events<" not in dense.source


def test_random_draws_in_pathway_code_lower_to_the_edge_indexed_counter_rng():
    """rand() lowers to the counter RNG in neuron code (indexed by the neuron) and in pathway code
    (indexed by the edge, executor.rs:5071-5074): procedural rows are in edge order and index it
    directly, an explicit layout (rows sorted by source and target block) reads each row's edge
    index from a table; such a group is ordered, never counted.  A scalar statement of neuron code
    draws with index 0 on the device, once per tick (with rand() and arithmetic only: a host libm
    transcendental could differ by an ulp); a pathway's scalar statements are rejected before
    device work."""
    plan = _generate(models.poisson_network(300, 500, indegree=20, steps=20))
    assert "atlas::counter_uniform(1729ull, 0ull, (u64)tick, (u64)(i))" in plan.source
    doc = models.poisson_network(300, 500, indegree=20, steps=20)
    value = doc["definition"]["synapses"][0]["code_objects"][0]["vector"][0]["value"]["arg"]
    value["right"] = {"op": "mul", "left": value["right"], "right": models.rand(1)}
    protocol.seal(doc)
    plan = _generate(doc)
    path = plan.pathways[0]
    assert path.random and not engine.counting_group([path])
    table = path.buffers["edge_id"]
    assert (f"atlas::counter_uniform(1729ull, 1ull, (u64)tick, (u64)(atlas::buf<const u32>(tab, {table})[row]))"
            in plan.source)
    np.testing.assert_array_equal(plan.buffers[table].init, path.order.astype(np.uint32))
    plan = _generate(models.random_pathway_network(procedural=True))
    assert "edge_id" not in plan.pathways[0].buffers
    assert "atlas::counter_uniform(1729ull, 1ull, (u64)tick, (u64)(row))" in plan.source
    plan = _generate(models.random_pathway_network(draw="randn"))
    assert "atlas::counter_normal(1729ull, 1ull, (u64)tick, (u64)(atlas::buf<const u32>" in plan.source
    plan = _generate(nets.shared_draw_network(100, steps=5))
    assert "atlas::counter_uniform(5ull, 2ull, (u64)tick, (u64)(0))" in plan.source
    assert "atlas::counter_uniform(5ull, 3ull, (u64)tick, (u64)(i))" in plan.source
    shared = nets.shared_draw_network(100, steps=5)
    update = next(c for c in shared["definition"]["populations"][0]["code_objects"] if c["kind"] == "state_update")
    update["scalar"][0]["value"] = {"op": "exp", "arg": models.rand(2)}
    protocol.seal(shared)
    with pytest.raises(engine.UnsupportedModel, match="rand\\(\\) and arithmetic"):
        _generate(shared)
    scalar = models.random_pathway_network()
    code = scalar["definition"]["synapses"][0]["code_objects"][0]
    code["scalar"] = [models.stmt("_s", "f64", models.rand(3))]
    protocol.seal(scalar)
    with pytest.raises(engine.UnsupportedModel):
        _generate(scalar)


def test_plan_structure_of_the_fixture(fixture_doc):
    plan = _generate(fixture_doc)
    assert [p.count for p in plan.populations] == [80, 20]
    assert plan.steps == 256 and plan.dt == 1e-4
    assert len(plan.pathways) == 4
    assert all(path.topology[0] == "explicit" for path in plan.pathways)
    # per-edge delays 1..4 become delay groups
    assert sorted({int(d) for path in plan.pathways for d in path.dvals}) == [1, 2, 3, 4]


def test_delay_zero_shifts_the_deliveries_one_launch_later():
    """A delay-0 pathway needs every block's spikes of the tick: each tick's launch delivers the
    previous tick, then updates its own, and an epilogue launch delivers the run's last tick; the
    spike ring holds one more tick."""
    plan = _generate(models.cuba_network(1000, steps=10))
    assert plan.kernels == ["atlas_tick", "atlas_tick_deliver"]
    assert [k for k, *_ in plan.launches] == [0] and [k for k, *_ in plan.epilogue] == [1]
    assert plan.populations[0].ring == 2
    head = plan.source[plan.source.index('void __launch_bounds__(256) atlas_tick('):]
    head = head[:head.index("extern")] if "extern" in head else head
    # the block's states load first; the previous tick's counts are applied to them in registers
    assert plan.populations[0].fused_split
    assert (head.index("atlas::phase_a_load<Pop0>(tab, blk, st)") < head.index("atlas::deliver<Group0, false>(tab, tick_prev")
            < head.index("atlas::pre_apply<Pop0, Fused0>(tab, tick_prev, t_prev") < head.index("atlas::phase_a_run<Pop0>(tab, tick, t"))
    assert f"if (tick > {plan.start_tick}LL)" in head
    plan = _generate(models.cuba_network(1000, steps=10, delay_ticks=1))
    assert plan.kernels == ["atlas_tick"] and not plan.epilogue and plan.populations[0].ring == 2


def test_reset_fusion_decision():
    plan = _generate(models.cuba_network(3000, indegree=50, delay_ticks=1, steps=10))
    assert plan.populations[0].reset_fused          # reset writes v, deliveries write ge/gi
    plan = _generate(models.delta_lif_network(3000, indegree=50, steps=10))
    assert not plan.populations[0].reset_fused      # deliveries write v: reset must follow them
    assert [[p.index for p in g] for g in plan.groups] == [[0], [1]]


def test_explicit_layout_rows_and_segments(fixture_doc):
    plan = engine.lower(fixture_doc)
    for path in plan.pathways:
        nb = plan.populations[path.target].blocks
        row_target, seg, order = engine.explicit_layout(path, nb, plan.shape.block)
        _, src, tgt = path.topology
        assert sorted(order.tolist()) == list(range(path.edge_count))
        np.testing.assert_array_equal(row_target, (tgt + path.tstart)[order])
        D = len(path.dvals)
        delays = path.delays if path.delays.size == path.edge_count else np.full(path.edge_count, path.dvals[0])
        seg = seg.reshape(path.scount * D, nb + 1).astype(np.int64)
        assert seg[0, 0] == 0 and seg[-1, -1] == path.edge_count
        assert np.all(np.diff(seg, axis=1) >= 0)
        np.testing.assert_array_equal(seg[1:, 0], seg[:-1, -1])
        for s in range(path.scount):
            for g in range(D):
                for b in range(nb):
                    rows = np.arange(seg[s * D + g, b], seg[s * D + g, b + 1])
                    edges = order[rows]
                    assert np.all(src[edges] == s)
                    assert np.all(delays[edges] == path.dvals[g])
                    assert np.all(row_target[rows] // plan.shape.block == b)
                    key = row_target[rows].astype(np.int64) * path.edge_count + edges
                    assert np.all(np.diff(key) > 0)     # target ascending, then edge ascending


def test_initial_until_matches_brute_force():
    """First tick from which timestep(t - lastspike, dt) >= period holds (executor.rs:4045-4058)."""
    dt, period, start = 1e-4, 50, 0
    rng = np.random.default_rng(3)
    last = np.concatenate([[-1e4, 0.0, -dt, -49 * dt, -50 * dt, -51 * dt],
                           -rng.integers(0, 60, 200) * dt, -rng.random(200) * 60 * dt])
    got = engine.initial_until(last, start, dt, period)
    for value, until in zip(last.tolist(), got.tolist()):
        ok = [math.floor((tick * dt - value + 1e-3 * dt) / dt) >= period for tick in range(start, 200)]
        first = next((k for k, flag in enumerate(ok) if all(ok[k:])), None)
        assert until == start + first


def _document_with(document, mutate):
    doc = copy.deepcopy(document)
    mutate(doc)
    return protocol.seal(doc)


def test_unsupported_models_are_rejected_before_any_device_work():
    base = models.cuba_network(500, steps=10)

    def sin_in_vector(doc):
        # sin has no shared implementation with matching CPU/GPU bits
        pop = doc["definition"]["populations"][0]
        update = next(c for c in pop["code_objects"] if c["kind"] == "state_update")
        update["vector"][1]["value"] = {"op": "f64_to_f32", "arg": {"op": "sin", "arg": {"op": "load", "name": "taue"}}}

    def second_clock(doc):
        doc["definition"]["clocks"].append({"name": "other", "dt": models.f64_hex(2e-4)})
        doc["definition"]["populations"][0]["clock"] = 1

    def unknown_topology(doc):
        doc["instance"]["synapses"][0]["topology"] = {"kind": "bernoulli_procedural"}

    for mutate in (sin_in_vector, second_clock, unknown_topology):
        with pytest.raises(engine.UnsupportedModel):
            _generate(_document_with(base, mutate))


def test_tampered_document_is_rejected():
    doc = models.cuba_network(500, steps=10)
    doc["run"]["clocks"][0]["steps"] = 11
    with pytest.raises(protocol.ProtocolError):
        engine.lower(doc)


def test_procedural_seed_and_initializer_streams():
    """connect_fixed_indegree seeds (device.py:299-302) and streams 2 + 2k (export.py:2386-2403)."""
    doc = models.cuba_network(5000, indegree=100, steps=10)
    topo = [s["topology"] for s in doc["instance"]["synapses"]]
    assert [t["seed"] for t in topo] == [(1729 ^ (k * 0x9E3779B97F4A7C15)) & (2**64 - 1) for k in (1, 2)]
    assert [t["indegree"] for t in topo] == [80, 20]
    assert [t["edge_count"] for t in topo] == [80 * 5000, 20 * 5000]


def test_packed_documents_lower_to_the_same_plan():
    """In-memory packed arrays (numpy in place of hex lists) give the same device buffers."""
    hexed = models.plastic_network(3000, indegree=100, steps=20, packed=False)
    packed = models.plastic_network(3000, indegree=100, steps=20, packed=True)
    assert "protocol" not in packed
    a, b = _generate(hexed), engine.lower(packed, verify_envelope=False)
    engine.allocate(b)
    engine.generate(b, native.device_header_text())
    assert a.source == b.source
    assert [x.name for x in a.buffers] == [x.name for x in b.buffers]
    for x, y in zip(a.buffers, b.buffers):
        assert x.nbytes == y.nbytes
        if x.init is not None:
            np.testing.assert_array_equal(np.asarray(x.init).view(np.uint8), np.asarray(y.init).view(np.uint8),
                                          err_msg=x.name)


def test_fixed_indegree_sample_is_distinct_and_source_major():
    rng = np.random.default_rng(4)
    src, tgt = models.fixed_indegree_sample(rng, 300, 500, 40)
    assert src.size == 500 * 40
    assert np.all(np.diff(src) >= 0)
    for t in range(0, 500, 37):
        assert np.unique(src[tgt == t]).size == 40
    assert np.array_equal(np.bincount(tgt, minlength=500), np.full(500, 40))


def _continuation_doc(document, boundary):
    """The second segment of `document` split at `boundary`, its first run by the oracle."""
    from atlas_hip.continuation import continuation, first_segment
    from atlas_hip.results import result_from_dump
    from oracle import oracle
    steps = protocol.load(document)["run"]["clocks"][0]["steps"]
    first = first_segment(document, boundary)
    run = oracle.run(first, shared_math=True, lift_recording_budget=True)
    return continuation(first, result_from_dump(run.results, protocol.load(first)), steps - boundary)


@pytest.mark.parametrize("name", ["fixture", "stdp"])
def test_pending_event_tables(name, fixture_doc):
    """A continuation's pending events, per (tick offset, target block) in the order given:
    uniform-delay events expand to their source's out-edges, edges ascending; every entry
    names the row of its edge and the block-local target; on_post events name neurons."""
    document = {"fixture": lambda: _continuation_doc(fixture_doc, 128),
                "stdp": lambda: _continuation_doc(nets.stdp_network(64, 8, 400), 200)}[name]()
    plan = _generate(document)
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000
    block = plan.shape.block
    pending_groups = [g for g in plan.groups if g[0].pending_ticks]
    assert pending_groups
    for group in pending_groups:
        offsets, entries, ticks = engine.pending_layout(plan, group)
        tb = plan.populations[group[0].target].blocks
        expected = {}
        for p, path in enumerate(group):
            if path.pending is None:
                continue
            _, src, tgt = path.topology
            row_of_edge = np.empty(path.edge_count, np.int64)
            row_of_edge[path.order] = np.arange(path.edge_count)
            for k, item, in zip(*path.pending[:2]):
                edges = np.flatnonzero(np.asarray(src) == item) if path.pending[2] else [item]
                for edge in edges:
                    target = int(tgt[edge]) + path.tstart
                    expected.setdefault((int(k), target // block), []).append(
                        (int(row_of_edge[edge]), target % block | p << 16))
        for k in range(ticks):
            for b in range(tb):
                got = entries[offsets[k * tb + b]:offsets[k * tb + b + 1]].tolist()
                assert [tuple(e) for e in got] == expected.get((k, b), [])
    if name == "stdp":
        post = plan.post_paths[0]
        assert post.pending_ticks and "deliver_post_pending<" in plan.source
        offsets, ids, ticks = engine.post_pending_layout(plan, post)
        k, items, _ = post.pending
        assert sorted(ids.tolist()) == sorted((items + post.pre.tstart).tolist())


def test_pending_events_are_checked():
    """model.rs:4322-4338 (ordered, inside the run, items in range); a counting group of one
    delay lists pending sources per tick; an on_post neuron may not repeat within one tick."""
    def with_pending(document, synapse, pathway, events):
        doc = copy.deepcopy(protocol.load(document, verify_envelope=False))
        doc.pop("protocol", None)
        doc["instance"]["synapses"][synapse]["pathways"][pathway]["pending"] = events
        return protocol.seal(doc)
    cuba = models.cuba_network(500, steps=50, delay_ticks=3)
    engine.lower(with_pending(cuba, 0, 0, [{"delivery_tick": 1, "item": 3}, {"delivery_tick": 2, "item": 3}]))
    for events in ([{"delivery_tick": 2, "item": 0}, {"delivery_tick": 1, "item": 0}],
                   [{"delivery_tick": 50, "item": 0}], [{"delivery_tick": 1, "item": 500}]):
        with pytest.raises(engine.UnsupportedModel, match="invalid pending"):
            engine.lower(with_pending(cuba, 0, 0, events))
    # a procedural (counting, one-delay) group takes its pending events as pending sources
    procedural = models.cuba_network(5000, indegree=100, delay_ticks=3, steps=50)
    plan = _generate(with_pending(procedural, 0, 0, [{"delivery_tick": 1, "item": 0}, {"delivery_tick": 1, "item": 7}]))
    assert plan.groups[0][0].pending_sources and plan.groups[0][0].pending_ticks == 2
    offsets, ids, ticks = engine.pending_source_layout(plan, plan.groups[0])
    assert offsets.tolist() == [0, 0, 2] and ids.tolist() == [0, 7] and ticks == 2
    stdp = nets.stdp_network(64, 8, 50)
    with pytest.raises(engine.UnsupportedModel, match="repeat a neuron"):
        engine.lower(with_pending(stdp, 0, 1, [{"delivery_tick": 1, "item": 5}, {"delivery_tick": 1, "item": 5}]))


def test_binary_csr_lowers_to_the_explicit_layout(tmp_path):
    """A binary_csr topology lowers to the same edges (source-major file order) and per-edge
    parameter as the explicit document it came from, and its module compiles."""
    from atlas_hip.engine import decode_array
    doc, (offsets, targets, multiplicity) = models.binary_csr_example()
    binary = models.to_binary_csr(doc, 0, tmp_path / "graph.b2csr")
    plan = _generate(binary)
    path = plan.pathways[0]
    assert path.topology[0] == "explicit"
    assert path.topology[1].tolist() == np.repeat(np.arange(4), np.diff(offsets)).tolist()
    assert path.topology[2].tolist() == targets.tolist()
    assert path.edge_params["multiplicity"][1].tolist() == multiplicity.tolist()
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000
    # the declaration is checked: a column left unmapped
    inner = protocol.load(binary, verify_envelope=False)
    inner.pop("protocol", None)
    inner["instance"]["synapses"][0]["topology"]["initializers"] = {}
    with pytest.raises(engine.UnsupportedModel, match="binary CSR mapping"):
        engine.lower(protocol.seal(inner))


def test_rate_monitors_are_a_layout_over_the_spike_monitor():
    """A PopulationRateMonitor (model.rs:3379-3386) needs the spike monitor and changes nothing
    the engine or the oracle computes; without a spike monitor it is rejected."""
    from oracle import oracle
    base = protocol.load(models.cuba_network(500, steps=40), verify_envelope=False)
    base.pop("protocol", None)
    doc = copy.deepcopy(base)
    doc["definition"]["populations"][0]["rate_monitors"] = [{"name": "ratemonitor", "dtype": "f64"}]
    plain, rated = protocol.seal(copy.deepcopy(base)), protocol.seal(doc)
    engine.lower(rated)
    assert oracle.run(plain).results == oracle.run(rated).results
    doc["definition"]["populations"][0]["spike_monitor"] = None
    with pytest.raises(engine.UnsupportedModel, match="rate monitor"):
        engine.lower(protocol.seal(doc))


def test_executor_rejects_modes_it_does_not_implement():
    """As CudaExecutor (cuda.py:60-61, 91-92): numeric modes other than float32 and a supplied
    plan raise before any device work."""
    from atlas_hip.executor import HipExecutor, PlanValidationError
    doc = models.cuba_network(200, steps=5)
    for kwargs in ({"numeric_mode": "float64"}, {"numeric_mode": "reference"}, {"plan": object()}):
        with pytest.raises(PlanValidationError):
            HipExecutor(doc, **kwargs)


def test_persistent_eligibility():
    """Persistent launches are planned for one population whose deliveries are one counting group of
    one delay through slot tables, with a fused reset, no monitors reading states and at least 16
    blocks: config 3 (delay 1) and configs 1 and 2 (delay 0, 16 blocks of 256)."""
    big = models.cuba_network(100_000, indegree=100, delay_ticks=1, steps=5)
    plan = _generate(big)
    assert plan.persistent is not None and "atlas_run" in plan.kernels
    assert "persistent_run<" in plan.source and plan.populations[0].ring == 4   # 2 d + 2 ticks
    assert _generate(models.cuba_network(100_000, indegree=100, delay_ticks=3, steps=5)).persistent is not None
    config1 = _generate(models.cuba_network(4000, steps=5))             # delay 0, 16 blocks, overlapping sources
    assert config1.persistent is not None and config1.split and "DISJOINT = false" in config1.source
    assert config1.populations[0].ring == 3                             # one more for the split launches
    assert _generate(models.cobahh_network(4000, steps=5)).persistent is not None
    assert _generate(models.cuba_network(3000, steps=5)).persistent is None      # 12 blocks
    # the plastic network's queued, on_post and multi-delay groups keep one launch per tick
    assert _generate(models.plastic_network(5000, steps=5, packed=False)).persistent is None


def test_weighted_network_runs_the_split_loop_through_edge_buckets():
    """An ordered group (a float32 weight per synapse, drawn from the edge id) of one delay >= 1 in
    4096-neuron blocks runs the split persistent loop through edge-keyed buckets: row slots (the
    first row in every slot), Group::edge_value selecting the pathway's initializer constants,
    Fused::apply_edge, and the LDS the loop's other arrays leave for the events (under 160 KB in
    all); the module compiles.  With 256-neuron blocks (no split loop), delay 0 or synapse states
    the plan keeps one launch per tick."""
    shape = engine.choose_shape(1_000_000, 1)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=5, weight_scale=0.0116, edge_weights=True)
    plan = engine.lower(doc, shape=shape)
    engine.allocate(plan)
    engine.generate(plan, native.device_header_text())
    assert plan.persistent is not None and plan.populations[0].fused_edges
    assert all(path.row_slots and "slot" in path.buffers for path in plan.pathways)
    assert "EDGE_SLOTS = true" in plan.source and "persistent_run_split<" in plan.source
    assert f"#define ATLAS_EDGE_NODES {plan.edge_nodes}u" in plan.source and plan.edge_nodes > 4800
    assert "atlas::edge_uniform(seed, stream, (u64)row, lo, hi)" in plan.source
    # the LDS the split loop's struct takes with the buckets of both parities (engine.LDS_BYTES at most)
    words = 2 * (4096 + 64 + 4) + 6 * plan.edge_nodes
    assert 4 * words + 4 * 8 * 256 + 4 * 8 * 64 + 64 * 4 + 24 + 64 * 8 + 4 * 2 * 16 * 2 <= engine.LDS_BYTES
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000
    assert _generate(doc).persistent is None                       # 256-neuron blocks: 391 blocks
    zero = engine.lower(models.cuba_network(100_000, indegree=100, delay_ticks=0, steps=5, edge_weights=True),
                        shape=shape)
    engine.allocate(zero)
    engine.generate(zero, native.device_header_text())
    assert zero.persistent is None and not any(path.row_slots for path in zero.pathways)


@pytest.mark.parametrize("kind,kept,dropped", [("overflow", ["u3"], ["u2"]), ("clip", ["u4", "u6"], ["u2", "u3", "u5"]),
                                               ("divisor", ["u4", "u6"], ["u2", "u3", "u5"]),
                                               ("exp", ["u5", "u7"], ["u2", "u3", "u4", "u6"])])
def test_finiteness_checks_implied_by_a_later_one_are_dropped(kind, kept, dropped):
    """A non-finite operand of +, -, *, a dividend, f32 rounding or negation makes the result
    non-finite, so the result's check (same guard) implies the operand's; the operands of a clip,
    a divisor and exp keep their own (their results can be finite)."""
    src = _generate(nets.nonfinite_network(kind, 4)).source
    step = src[src.index("static bool step"):src.index("return fired")]
    for var in kept:
        assert f"atlas::finite({var}, fault);" in step, (kind, var)
    for var in dropped:
        assert f"atlas::finite({var}, fault);" not in step and f"finiteness of {var} checked through" in step


def test_guarded_checks_are_not_implied_by_unguarded_ones():
    """The CUBA update: the refractory-guarded chain keeps one check, on its rounded result, under
    the guard; the unguarded decays keep theirs."""
    src = _generate(models.cuba_network(1000, steps=10)).source
    step = src[src.index("static bool step"):src.index("return fired")]
    guarded = [line for line in step.splitlines() if "atlas::finite(" in line and "!= 0.0)" in line]
    unguarded = [line for line in step.splitlines() if "atlas::finite(" in line and "!= 0.0)" not in line]
    rounded = next(line.split()[2] for line in step.splitlines() if "= (double)(float)(" in line)
    assert len(guarded) == 1 and f"atlas::finite({rounded}, fault)" in guarded[0]
    assert len(unguarded) == 3   # the two decays and the reset value


def test_host_prepared_topologies_equal_the_oracle():
    """The product's host materialisation of procedural projections (atlas_prepare_*) against the
    oracle's restatement, which the reference test pins (test_oracle.py): edges and initializer
    values bit for bit, and the reference's messages for invalid specifications."""
    for sources, targets, k, seed in [(8, 5, 3, nets.INIT_SEED), (1000, 700, 37, 99), (20_000, 300, 1000, 5)]:
        got, want = native.prepare_fixed_indegree(sources, targets, k, seed), oracle.fixed_indegree(sources, targets, k, seed)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    for sources, targets, edges, seed in [(8, 5, 257, nets.INIT_SEED), (1000, 700, 50_000, 3)]:
        got, want = native.prepare_fixed_total(sources, targets, edges, seed), oracle.fixed_total(sources, targets, edges, seed)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    assert np.array_equal(native.prepare_initializer(0, 5000, 7, 2, -0.5, 0.25), oracle.uniform(5000, 7, 2, -0.5, 0.25))
    assert np.array_equal(native.prepare_initializer(1, 5000, 7, 4, 1.0, 2.0, 1.5, 0.5),
                          oracle.clipped_normal(5000, 7, 4, 1.5, 0.5, 1.0, 2.0))
    assert np.array_equal(native.prepare_initializer(1, 5000, 7, 4, 0.0, 0.0, 1.5, 0.5, False, False),
                          oracle.clipped_normal(5000, 7, 4, 1.5, 0.5))
    with pytest.raises(native.PrepareError, match="invalid fixed-indegree"):
        native.prepare_fixed_indegree(3, 5, 4, 1)
    with pytest.raises(native.PrepareError, match="invalid fixed-total"):
        native.prepare_fixed_total(3, 5, 0, 1)
    with pytest.raises(native.PrepareError, match="invalid uniform"):
        native.prepare_initializer(0, 4, 1, 2, 1.0, 0.5)
    with pytest.raises(native.PrepareError, match="rejection limit"):
        native.prepare_initializer(1, 4, 1, 2, 5.0, 6.0, 0.0, 1e-9)


def test_procedural_projections_with_initializers_lower_as_explicit():
    """Fixed-total rules and projections with delay initializers or clipped-normal per-edge
    initializers are materialised on the host (the reference's GPU preparation) and lowered as
    explicit topologies; delays are floor(delay / dt + 0.5) of the initializer's values
    (executor.rs:86-90).  A fixed in-degree projection whose only initializers are uniform stays a
    device topology, its values drawn from the row (= edge id) where read."""
    for kind in ("total", "indegree"):
        for distribution in ("uniform", "normal"):
            doc = nets.initialization_network(kind, distribution)
            plan = engine.lower(doc)
            path = plan.pathways[0]
            reference = nets.initialization_endpoints(kind)
            assert path.topology[0] == "explicit"
            assert np.array_equal(path.topology[1], reference[:, 0]) and np.array_equal(path.topology[2], reference[:, 1])
            count = len(reference)
            delays = np.array([3 * nets.initialization_uniform(4, e) if distribution == "uniform"
                               else nets.initialization_normal(4, e, 1.5, .5, 0, 3) for e in range(count)])
            assert np.array_equal(path.delays, np.floor(delays + .5).astype(np.int64))
            assert "w" in path.edge_params
    plan = engine.lower(models.cuba_network(4000, indegree=100, steps=10))
    assert plan.pathways[0].topology[0] == "fixed_indegree"   # no initializers: built on the device
    plan = engine.lower(models.cuba_network(4000, indegree=100, steps=10, weight_scale=0.5, edge_weights=True))
    we, wi = models.CUBA["we"] * 0.5, models.CUBA["wi"] * 0.5
    by_name = {path.name: path for path in plan.pathways}
    for name, (low, high) in (("synapses_pre", (0.5 * we, 1.5 * we)), ("synapses_1_pre", (1.5 * wi, 0.5 * wi))):
        path = by_name[name]
        assert path.topology[0] == "fixed_indegree" and path.edge_params == {"w": ("f32", None)}
        seed, stream, lo, hi = path.edge_gen["w"]
        assert (stream, lo, hi) == (2, low, high) and seed == path.topology[2] & (2**64 - 1)
        assert engine._edge_param_expr(path, "w").startswith(f"atlas::edge_uniform({seed}ull, 2ull, (u64)row, ")


def test_summed_variables_and_clock_driven_states_lower_before_the_tick():
    """Summed variables and the clock-driven synapse state update run as their own launches
    before each tick's launch, in schedule order: (groups, -1) summed variables first, then the
    synapse state update (order 0, which commutes with the neuron updates), and a summed variable
    over a partial range (order 0) by name after it.  The module compiles; such plans are never
    persistent."""
    plan = _generate(nets.summed_network(2000, steps=5))
    assert [(c.kind, c.state, c.to_pre) for c in plan.synapse_codes] == [
        ("summed", "I", False), ("summed", "J", True), ("update", "", False)]
    assert plan.pathways[0].topology[0] == "explicit"        # the edges are needed on the host
    assert [plan.kernels[k] for k, *_ in plan.launches] == ["atlas_syn0", "atlas_syn1", "atlas_syn2", "atlas_tick"]
    assert plan.launches[2][1] * plan.launches[2][2] >= 2000 * 100 and plan.persistent is None
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000
    plan = _generate(nets.summed_pin_network([0, 1], [1, 1], [0.25, 0.5], target_range=(2, 4)))
    assert [(c.kind, c.state) for c in plan.synapse_codes] == [("summed", "J"), ("update", ""), ("summed", "I")]
    offsets, rows = engine.endpoint_layout(plan.pathways[0], to_pre=False)
    assert offsets.tolist() == [0, 0, 2] and sorted(rows.tolist()) == [0, 1]


def test_summed_variables_with_delay_zero_run_between_the_previous_deliveries_and_the_update():
    """With a delay-0 pathway a tick's deliveries need every block's spikes of that tick, so they run
    one launch later; synapse programs of the groups slot must see them and come before the update.
    The tick is then three launch kinds: the previous tick's deliveries and resets, the synapse
    programs, the update (the reference's order: synapses and resets of t - 1, groups of t), and
    the epilogue delivers the last tick."""
    plan = _generate(nets.summed_network(500, indegree=10, steps=5, delay_ticks=0))
    assert [plan.kernels[k] for k, *_ in plan.launches] == [
        "atlas_tick_deliver_previous", "atlas_syn0", "atlas_syn1", "atlas_syn2", "atlas_tick"]
    assert [plan.kernels[k] for k, *_ in plan.epilogue] == ["atlas_tick_deliver"]
    assert plan.persistent is None
    head = plan.source[plan.source.index("atlas_tick_deliver_previous("):]
    assert f"if (tick > {plan.start_tick}LL)" in head[:head.index("extern")]
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000


def test_unsupported_summed_variable_placements_are_rejected():
    """A state monitor recording the summed state (it records before the groups slot) and a
    summed variable scheduled after its population's update are refused with the reason."""
    doc = nets.summed_network(500, indegree=10, steps=5)
    doc["definition"]["populations"][0]["monitor"]["variables"] = ["I"]
    doc["definition"]["populations"][0]["monitor"]["record"] = [0]
    with pytest.raises(engine.UnsupportedModel, match="state monitor recording a summed"):
        engine.lower(protocol.seal(doc))
    doc = nets.summed_network(500, indegree=10, steps=5)
    nodes = doc["definition"]["schedule"]["nodes"]
    summed = next(k for k, n in enumerate(nodes) if n["owner_kind"] == "synapse")
    update = next(k for k, n in enumerate(nodes) if n["owner_kind"] == "population" and n["operation"] == "code_object")
    nodes[summed], nodes[update] = nodes[update], nodes[summed]
    with pytest.raises(engine.UnsupportedModel, match="schedule order"):
        engine.lower(protocol.seal(doc))


def test_merged_clock_steps_follow_the_epsilon_rule():
    """Clocks of 0.1, 0.15 and 0.2 ms over 0.6 ms: each step advances every clock whose next
    tick time is within 1e-12 of the smallest dt of the earliest one, so 3 * 0.1 ms and 2 *
    0.15 ms (which differ in their last bits) share a step, and each clock stops at its own
    end.  Written out from the times 0, 0.1, 0.15, 0.2, 0.3, 0.4, 0.45, 0.5 ms."""
    table = engine.merged_clock_steps([(1e-4, 0, 6), (1.5e-4, 0, 4), (2e-4, 0, 3)])
    assert 3 * 1e-4 != 2 * 1.5e-4
    assert table.tolist() == [[0, 0, 0], [1, -1, -1], [-1, 1, -1], [2, -1, 1], [3, 2, -1], [4, -1, 2],
                              [-1, 3, -1], [5, -1, -1]]
    # every clock advances exactly its own steps, in order
    for c, count in enumerate((6, 4, 3)):
        ticks = table[:, c][table[:, c] >= 0]
        assert ticks.tolist() == list(range(count))
    # later starts and clocks that never coincide: 0.9, 1.0, 1.1, 1.2 ms
    table = engine.merged_clock_steps([(1e-4, 10, 2), (3e-4, 3, 2)])
    assert table.tolist() == [[-1, 3], [10, -1], [11, -1], [-1, 4]]


@pytest.mark.parametrize("seed", range(8))
def test_merged_clock_steps_order_every_tick_once(seed):
    """Random clocks (dt of 1..7 units of 0.05 ms, random starts and lengths): each clock advances
    exactly its own ticks in order, step times are strictly increasing, and every step advances
    exactly the clocks whose tick time is that step's time (times compared in integer units)."""
    rng = np.random.default_rng(seed)
    units = [int(u) for u in rng.integers(1, 8, rng.integers(2, 5))]
    clocks = [(u * 5e-5, int(rng.integers(0, 20)), int(rng.integers(1, 40))) for u in units]
    table = engine.merged_clock_steps(clocks)
    for c, (_, start, count) in enumerate(clocks):
        ticks = table[:, c][table[:, c] >= 0]
        assert ticks.tolist() == list(range(start, start + count))
    times = []
    for row in table:
        step = {int(row[c]) * units[c] for c in range(len(clocks)) if row[c] >= 0}
        assert len(step) == 1
        times.append(step.pop())
        # no clock that is still running has a tick at this time that the step leaves out
        for c, (_, start, count) in enumerate(clocks):
            if row[c] < 0:
                assert all(k * units[c] != times[-1] for k in range(start, start + count))
    assert all(a < b for a, b in zip(times, times[1:]))


def test_multiclock_network_lowers_to_one_table_driven_launch():
    """Three populations on three clocks lower to one atlas_tick per merged step: the plan's
    steps are the merged steps, each population keeps its clock's tick count, and the module
    (phase A on the population's clock, deliveries on the source's) compiles."""
    plan = _generate(nets.multiclock_network(600, steps=60))
    assert plan.multi_clock and plan.start_tick == 0 and plan.persistent is None
    assert [pop.clock for pop in plan.populations] == [0, 1, 2]
    assert [pop.steps for pop in plan.populations] == [60, 40, 30]
    assert plan.steps == plan.clock_table.shape[0] and plan.clock_table.shape[1] == 3
    assert [plan.end_tick(pop, plan.steps) for pop in plan.populations] == [60, 40, 30]
    assert "atlas::stage<Pop1>" in plan.source and "tick1 >= 0" in plan.source
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000


def test_multiclock_delay_zero_splits_each_step_into_updates_and_deliveries():
    """With a delay-0 pathway across clocks a step's deliveries need every block's spikes of the
    step: each merged step is two launches, the updates (and pushes) of the clocks that advance,
    then their deliveries, on_post pathways, resets and end code; no epilogue."""
    plan = _generate(nets.multiclock_network(600, steps=60, monitor=False, zero_delay=True))
    assert plan.split and plan.multi_clock
    assert [plan.kernels[k] for k, *_ in plan.launches] == ["atlas_tick", "atlas_tick_deliver"] and not plan.epilogue
    update = plan.source[plan.source.index("atlas_tick(const u64"):plan.source.index("atlas_tick_deliver(const u64")]
    deliver = plan.source[plan.source.index("atlas_tick_deliver(const u64"):]
    assert "atlas::phase_a<" in update and "atlas::deliver<" not in update and "reset_phase" not in update
    assert "atlas::deliver<" in deliver and "atlas::phase_a<" not in deliver and "reset_phase" in deliver
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000


def test_synapse_programs_across_clocks_run_on_their_own_clock():
    """With several clocks each synapse program launch reads its own clock's tick from the clock table
    and returns when that clock does not advance; a summed variable must run on the clock of the
    population it sets."""
    plan = _generate(nets.summed_multiclock_network(400, steps=20))
    assert plan.multi_clock and [(c.kind, c.code["clock"]) for c in plan.synapse_codes] == [
        ("summed", 1), ("summed", 0), ("update", 0)]
    head = plan.source[plan.source.index("atlas_syn0("):]
    head = head[:head.index("}")]
    assert f"atlas::buf<const i64>(tab, {plan.clock_buffer})[(u64)step * 2u + 1u]" in head and "if (tick < 0) return;" in head
    doc = nets.summed_multiclock_network(400, steps=20)
    node = next(n for n in doc["definition"]["schedule"]["nodes"] if n["owner_kind"] == "synapse"
                and doc["definition"]["synapses"][0]["code_objects"][n["item_index"]]["kind"] == "summed_variable")
    code = doc["definition"]["synapses"][0]["code_objects"][node["item_index"]]
    node["clock"] = code["clock"] = 1 - code["clock"]
    with pytest.raises(engine.UnsupportedModel, match="clock of the population it sets"):
        engine.lower(protocol.seal(doc))


def test_custom_events_lower_to_flags_and_a_generated_resets_slot():
    """Custom events (NeuronGroup events=..., run_on_event): each condition runs in the update's
    step on the updated states and leaves a flag per neuron; the resets slot runs the resets in
    schedule order (alpha, spike, zeta: names sort alpha before spike), the end-of-tick monitors
    and the event bitmaps; the spike reset is not fused and the plan is never persistent.  A
    condition reading refractoriness and end-of-tick monitors beside end-of-tick run_regularly
    code are rejected."""
    plan = _generate(nets.custom_event_network())
    pop = plan.populations[0]
    assert [e for e, _, _ in pop.custom_events] == ["alpha", "zeta"] and pop.reset_order == ["alpha", "spike", "zeta"]
    assert not pop.reset_fused and plan.persistent is None
    assert {"evt:0", "evt:1", "evrec:0", "evrec:1"} <= set(pop.buffers)
    assert "custom_phase(" in plan.source and "static constexpr bool CUSTOM = true;" in plan.source
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000
    doc = nets.custom_event_network()
    code = next(c for c in doc["definition"]["populations"][0]["code_objects"]
                if c["kind"] == "threshold" and c["event_name"] == "alpha")
    code["vector"][0]["value"] = models.op("and", code["vector"][0]["value"], models.ld("not_refractory"))
    code["effects"]["reads"] = sorted(set(code["effects"]["reads"]) | {"not_refractory"})
    with pytest.raises(engine.UnsupportedModel, match="refractoriness"):
        engine.lower(protocol.seal(doc))


def test_plastic_rows_are_ordered_by_target_and_keep_the_canonical_order():
    """The queued STDP pathway of a plastic network stores its rows by target: a target's
    incoming edges are one run of rows (the on_post pass reads them as one range), the rows of
    one target keep the source-major order (source, delay, edge) that queued events compare,
    and every out-edge position maps to the row of its own edge."""
    plan = _generate(models.plastic_network(1500, indegree=200, delays=(1, 5), steps=20, packed=False))
    path = next(p for p in plan.pathways if p.post_major)
    assert [p.index for p in plan.pathways if p.post_major] == [path.index] and path.index in plan.queues
    _, src, tgt = path.topology
    src, tgt = np.asarray(src, np.int64), np.asarray(tgt, np.int64)
    NB = plan.populations[path.target].blocks
    out_tgt, seg, order, out_row = engine.post_major_layout(path, NB, plan.shape.block)
    ref_tgt, ref_seg, out_order = engine.explicit_layout(path, NB, plan.shape.block)
    assert np.array_equal(out_tgt, ref_tgt) and np.array_equal(seg, ref_seg)
    assert np.array_equal(order[out_row], out_order)   # a position's row holds that position's edge
    assert np.all(np.diff(tgt[order]) >= 0)
    # within a target, rows ascend with the source-major positions
    position = np.empty(path.edge_count, np.int64)
    position[out_order] = np.arange(path.edge_count)
    by_target = np.lexsort((position, tgt))
    assert np.all(np.diff(np.argsort(order)[by_target])[np.diff(tgt[by_target]) == 0] > 0)
    offsets, rows = engine.post_layout(path)
    assert np.array_equal(rows, np.arange(path.edge_count))
    assert np.array_equal(np.repeat(np.arange(path.tcount), np.diff(offsets.astype(np.int64))), tgt[order])
    assert f"atlas::buf<const u32>(tab, {path.buffers['out_row']})[k]" in plan.source


def test_custom_event_routes_lower_to_event_rings():
    """A pathway on a custom event reads a ring of that event's fired neurons (published with the
    spikes, sized by its delays) and is never grouped with a spike pathway; a Synapses may hold
    several on_pre pathways: the synapse states live in the rows of the first that touches them,
    and the others that touch them reach those records through a row map and are never grouped
    with them."""
    plan = _generate(nets.custom_route_network())
    source = plan.populations[0]
    assert [(p.name, p.event) for p in plan.pathways] == [
        ("projection_alpha_path", "alpha"), ("projection_spike_path", "spike"), ("projection_zeta_path", "zeta")]
    assert source.event_rings == {0: 5, 1: 2} and {"ering_ids:0", "ering_cnt:1"} <= set(source.buffers)
    assert all(len(group) == 1 for group in engine.delivery_groups(plan))
    assert "publish_events(" in plan.source and "static constexpr bool EVENT_RINGS = true;" in plan.source
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000
    plan = _generate(nets.custom_route_network(mutable=True))
    owner, *sharers = plan.pathways
    assert owner.state_owner is None and "syn" in owner.buffers and "rec_row" not in owner.buffers
    assert [p.state_owner for p in sharers] == [owner, owner]
    assert all(p.buffers["syn"] == owner.buffers["syn"] for p in sharers)
    for p in sharers:   # a row's record holds that row's own edge
        rec = plan.buffers[p.buffers["rec_row"]].init
        np.testing.assert_array_equal(np.asarray(owner.order)[rec], p.order)
    assert f"atlas::buf<const u32>(tab, {sharers[0].buffers['rec_row']})[row]" in plan.source
    assert all(len(group) == 1 for group in engine.delivery_groups(plan))
    assert len(rtc.compile_source(plan.source, engine.COMPILE_OPTIONS)) > 1000


def test_event_conditions_outside_the_thresholds_slot_are_rejected():
    """A custom event scheduled at the end of the tick (set_event_schedule(..., when='end'); the
    reference test test_gpu_custom_events.py:110-128) would see the states after the resets: the
    engine, which evaluates every condition in the update's step, refuses it with the reason."""
    doc = copy.deepcopy(protocol.load(nets.custom_route_network(two_clocks=False)))
    doc.pop("protocol", None)
    d = doc["definition"]
    for node in d["schedule"]["nodes"]:
        if node["owner_kind"] == "population" and node["owner_index"] == 0 and node["operation"] == "code_object":
            code = d["populations"][0]["code_objects"][node["item_index"]]
            if code["kind"] == "threshold" and code.get("event_name") == "zeta":
                node["when"] = "end"
    with pytest.raises(engine.UnsupportedModel, match="threshold code outside the thresholds slot"):
        engine.lower(protocol.seal(doc))


def test_multiclock_restrictions_are_rejected():
    """A pathway scheduled on a clock other than its source's is refused with the reason."""
    doc = nets.multiclock_network(600, steps=60, monitor=False)
    node = next(n for n in doc["definition"]["schedule"]["nodes"] if n["owner_kind"] == "synapse")
    node["clock"] = (node["clock"] + 1) % 3
    with pytest.raises(engine.UnsupportedModel, match="clock of the population that triggers it"):
        engine.lower(protocol.seal(doc))


@pytest.mark.parametrize("dt,period,start", [(1e-4, 50, 0), (1e-4, 20, 987_654), (1.0 / 1024, 3, 5), (3e-4, 1, 123),
                                             (0.1e-3, 2, 10_000_000)])
def test_refractory_table_equals_the_recompute_search(dt, period, start):
    """The per-tick refractory deadlines a launch reads (the device search of refractory_until,
    vectorised) equal the first tick after the spike at which the reference's recompute
    ``timestep(tick dt - lastspike, dt) >= period`` holds, found by the independent search the
    engine uses for initial refractory states (initial_until)."""
    steps = 3000
    table = engine.refractory_table(start, steps, dt, dt, period)
    assert table is not None and table.dtype == np.int32
    for k in list(range(0, steps, 37)) + [steps - 1]:
        tick = start + k
        expected = engine.initial_until(np.array([tick * dt]), tick + 1, dt, period)[0]
        assert table[k] == expected, (tick, table[k], expected)
    assert engine.refractory_table(0, engine.UNTIL_TABLE_TICKS + 1, dt, dt, period) is None
