"""Persistent launches (one cooperative launch for many ticks, the block's states in registers,
the spike ring exchanged device-coherently across XCDs, a grid barrier between ticks) against
the CPU oracle and against one launch per tick: identical dumps, bit for bit."""
import numpy as np
import pytest

from atlas_hip import engine, models, protocol
from atlas_hip.executor import HipExecutor
from atlas_hip.models import hex_array
from atlas_hip.results import write_events, write_results
from oracle import oracle

pytestmark = pytest.mark.gpu


def run(doc, mode, monkeypatch, plain=False, **kwargs):
    monkeypatch.setenv("ATLAS_HIP_PERSISTENT", ("plain" if plain else "1") if mode == "persistent" else "0")
    with HipExecutor(doc, device=0, **kwargs) as ex:
        result = ex.run()
        assert result["hip_runtime"]["launch_mode"] == mode
        return write_results(ex.document, result), write_events(ex.document, result), result


def test_tenth_scale_persistent_equals_oracle_and_per_tick(monkeypatch):
    """Config 3's network at 100k neurons (in-degree 1000, 1e8 synapses), 150 ticks."""
    print("case: persistent scaled CUBA 100k x 1000, 150 ticks", flush=True)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=150, weight_scale=0.0116)
    expected = oracle.run(doc, lift_recording_budget=True)
    assert expected.synaptic_events > 1_000_000
    dump, events, result = run(doc, "persistent", monkeypatch, lift_recording_budget=True)
    assert dump == expected.results and events == expected.events
    assert result["hip_runtime"]["launches"] == 1
    tick_dump, tick_events, _ = run(doc, "per-tick", monkeypatch, lift_recording_budget=True)
    assert tick_dump == dump and tick_events == events


def test_plain_persistent_launches_equal_cooperative_ones(monkeypatch):
    """The same kernel issued as ordinary launches (the grid fits the device at once by its
    occupancy) gives the oracle's dump, over launches of 40 ticks."""
    print("case: plain persistent launches, scaled CUBA 100k x 1000, 120 ticks", flush=True)
    monkeypatch.setattr(engine, "PERSISTENT_TICKS", 40)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=120, weight_scale=0.0116)
    expected = oracle.run(doc, lift_recording_budget=True)
    dump, events, result = run(doc, "persistent", monkeypatch, plain=True, lift_recording_budget=True)
    assert result["hip_runtime"]["launches"] == 3
    assert dump == expected.results and events == expected.events


def test_persistent_run_split_over_launches(monkeypatch):
    """A run of 150 ticks in launches of 37 ticks (the states pass through memory between them)."""
    print("case: persistent scaled CUBA 100k x 1000, launches of 37 ticks", flush=True)
    monkeypatch.setattr(engine, "PERSISTENT_TICKS", 37)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=150, weight_scale=0.0116)
    expected = oracle.run(doc, lift_recording_budget=True)
    dump, events, result = run(doc, "persistent", monkeypatch, lift_recording_budget=True)
    assert result["hip_runtime"]["launches"] == 5
    assert dump == expected.results and events == expected.events


def test_persistent_synchronous_burst(monkeypatch):
    """Every neuron starts above threshold: all 100k fire at tick 0 (256 per block, so the ring
    records' first 7 ids and the id lists are both read), then 1e8 events arrive at tick 1."""
    print("case: persistent burst 100k x 1000, 30 ticks", flush=True)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=30, weight_scale=0.0116)
    doc["instance"]["populations"][0]["initial_state"]["v"] = hex_array(np.full(100_000, -0.0495), "f32")
    protocol.seal(doc)
    expected = oracle.run(doc, lift_recording_budget=True)
    assert expected.synaptic_events >= 100_000 * 1000
    dump, events, _ = run(doc, "persistent", monkeypatch, lift_recording_budget=True)
    assert dump == expected.results and events == expected.events


def test_large_blocks_with_long_segments_equal_oracle_and_per_tick(monkeypatch):
    """280,000 neurons (one population of at least 64 x 4096) take 4096-neuron blocks of 1024
    work-items, one workgroup per CU; at in-degree 1000 a (source, block) segment holds 14.6
    targets on average, so about 40% exceed a slot's 15 inline targets and are read from the
    row table.  100 ticks: the persistent launch equals the oracle and one launch per tick."""
    print("case: persistent 280k x 1000 in 4096-neuron blocks, 100 ticks", flush=True)
    doc = models.cuba_network(280_000, indegree=1000, delay_ticks=1, steps=100, weight_scale=0.0116)
    expected = oracle.run(doc, lift_recording_budget=True)
    assert expected.synaptic_events > 1_000_000
    plan = engine.lower(doc)
    assert plan.shape.block == 4096 and plan.shape.wg == 1024 and plan.total_blocks == 69
    dump, events, result = run(doc, "persistent", monkeypatch, lift_recording_budget=True)
    assert dump == expected.results and events == expected.events
    tick_dump, tick_events, _ = run(doc, "per-tick", monkeypatch, lift_recording_budget=True)
    assert tick_dump == dump and tick_events == events


def test_large_block_burst_reads_long_segments(monkeypatch):
    """100k neurons forced into 25 blocks of 4096 (in-degree 1000: about 41 targets per segment,
    nearly every slot read from the row table), every neuron firing at tick 0 so that 1e8
    events arrive at tick 1, over 20 ticks: equal to the oracle."""
    print("case: persistent burst 100k x 1000 in 4096-neuron blocks, 20 ticks", flush=True)
    monkeypatch.setattr(engine, "PERSISTENT_MIN_BLOCKS", 16)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=1, steps=20, weight_scale=0.0116)
    doc["instance"]["populations"][0]["initial_state"]["v"] = hex_array(np.full(100_000, -0.0495), "f32")
    protocol.seal(doc)
    expected = oracle.run(doc, lift_recording_budget=True)
    assert expected.synaptic_events >= 100_000 * 1000
    dump, events, _ = run(doc, "persistent", monkeypatch, lift_recording_budget=True,
                          shape=engine.Shape(4096, 1024, 2, 11))
    assert dump == expected.results and events == expected.events


@pytest.mark.parametrize("model,ticks", [("cuba", 10_000), ("cobahh", 10_000)])
def test_delay_zero_persistent_equals_oracle_and_per_tick(monkeypatch, model, ticks):
    """Configs 1 and 2 (4000 neurons, Bernoulli p = 0.02, delay 0; 16 blocks of 256): each tick's
    deliveries follow its own publication and barrier inside the persistent launch.  CUBA's two
    pathways share the population as source range, so each fired source loads one slot per
    pathway.  Equal to the oracle and to one launch per tick (which delivers the previous tick
    first and the last tick in an epilogue)."""
    print(f"case: persistent delay 0, {model} 4000, {ticks} ticks", flush=True)
    doc = (models.cuba_network(4000, steps=ticks) if model == "cuba" else models.cobahh_network(4000, steps=ticks))
    # COBAHH in the oracle's libm mode: for this network its dump equals the shared-math mode's
    # (test_gpu_parity.py compares the device with the shared-math mode over the same ticks)
    expected = oracle.run(doc)
    dump, events, result = run(doc, "persistent", monkeypatch)
    assert result["hip_runtime"]["launches"] == 1
    assert dump == expected.results and events == expected.events
    tick_dump, tick_events, _ = run(doc, "per-tick", monkeypatch)
    assert tick_dump == dump and tick_events == events


def test_full_size_persistent_equals_per_tick(monkeypatch):
    """Config 3 at its full size (1M neurons, 1e9 synapses), 60 ticks: the persistent launch and one
    launch per tick give the same raster, states and event counts."""
    print("case: persistent scaled CUBA 1M x 1000, 60 ticks", flush=True)
    doc = models.cuba_network(1_000_000, indegree=1000, delay_ticks=1, steps=60, weight_scale=0.0116)
    dump, events, result = run(doc, "persistent", monkeypatch, lift_recording_budget=True, verify_envelope=False)
    assert len(result["populations"][0]["spike_ticks"]) > 10_000
    tick_dump, tick_events, _ = run(doc, "per-tick", monkeypatch, lift_recording_budget=True,
                                    verify_envelope=False)
    assert tick_dump == dump and tick_events == events


def test_persistent_longer_delay(monkeypatch):
    """Delay 3: each tick's deliveries wait for the spikes of tick - 3 only, so workgroups drift up
    to three ticks apart and the ring holds 2 d + 2 = 8 ticks."""
    print("case: persistent scaled CUBA 100k x 1000, delay 3, 200 ticks", flush=True)
    doc = models.cuba_network(100_000, indegree=1000, delay_ticks=3, steps=200, weight_scale=0.0116)
    expected = oracle.run(doc, lift_recording_budget=True)
    dump, events, result = run(doc, "persistent", monkeypatch, lift_recording_budget=True)
    assert dump == expected.results and events == expected.events


@pytest.mark.parametrize("delay,ticks,per_launch", [(0, 12_000, 12_000), (1, 20_000, 10_000)])
def test_runs_past_the_stamp_period_equal_oracle_and_per_tick(monkeypatch, delay, ticks, per_launch):
    """Ring words carry a 12-bit stamp that repeats every lcm(R, 4095) ticks: 4095 for delay 0's ring
    of 3 (here inside one launch of 12,000 ticks), 16,380 for delay 1's ring of 4 (here across two
    launches of 10,000).  Each publication clears the words its slot's previous tick wrote past its
    own count, so no stale word can carry the stamp a reader waits for.  CUBA 4000 (Bernoulli
    p = 0.02): equal to the oracle and to one launch per tick."""
    print(f"case: persistent delay {delay}, CUBA 4000, {ticks} ticks in launches of {per_launch}", flush=True)
    monkeypatch.setattr(engine, "PERSISTENT_TICKS", per_launch)
    doc = models.cuba_network(4000, steps=ticks, delay_ticks=delay)
    expected = oracle.run(doc)
    dump, events, result = run(doc, "persistent", monkeypatch)
    assert result["hip_runtime"]["launches"] == -(-ticks // per_launch)
    assert dump == expected.results and events == expected.events
    tick_dump, tick_events, _ = run(doc, "per-tick", monkeypatch)
    assert tick_dump == dump and tick_events == events


WEIGHTED_SHAPE = engine.choose_shape(1_000_000, 1)   # 4096-neuron blocks of 1024 work-items


def weighted(n, steps, **kwargs):
    return models.cuba_network(n, indegree=1000, delay_ticks=1, steps=steps, weight_scale=0.0116, edge_weights=True,
                               **kwargs)


def test_weighted_split_loop_equals_oracle_and_per_tick(monkeypatch):
    """Config 3's network with a float32 weight per synapse at 100k neurons in 4096-neuron blocks
    (25 workgroups of the split loop, edge-keyed lists applied in key order): the oracle's dump over
    150 ticks in one launch and in launches of 37 ticks, and the same as one launch per tick (the
    ordered LDS path)."""
    print("case: weighted split loop 100k x 1000, 150 ticks", flush=True)
    doc = weighted(100_000, 150)
    expected = oracle.run(doc, lift_recording_budget=True)
    assert expected.synaptic_events > 1_000_000
    monkeypatch.setenv("ATLAS_HIP_PERSISTENT", "1")
    with HipExecutor(doc, device=0, lift_recording_budget=True, shape=WEIGHTED_SHAPE) as ex:
        assert ex.plan.populations[0].fused_edges and "EDGE_SLOTS = true" in ex.plan.source
    dump, events, result = run(doc, "persistent", monkeypatch, lift_recording_budget=True, shape=WEIGHTED_SHAPE)
    assert result["hip_runtime"]["launches"] == 1
    assert dump == expected.results and events == expected.events
    monkeypatch.setattr(engine, "PERSISTENT_TICKS", 37)
    dump37, events37, result = run(doc, "persistent", monkeypatch, lift_recording_budget=True, shape=WEIGHTED_SHAPE)
    assert result["hip_runtime"]["launches"] == 5
    assert dump37 == dump and events37 == events
    tick_dump, tick_events, _ = run(doc, "per-tick", monkeypatch, lift_recording_budget=True, shape=WEIGHTED_SHAPE)
    assert tick_dump == dump and tick_events == events


def test_weighted_split_loop_burst_replays_per_tick(monkeypatch):
    """Every neuron starts above threshold, so 1e8 weighted events arrive at tick 1, 4e6 per block:
    more than a block's edge lists hold.  The launch reports it and the run is replayed with one
    launch per tick, equal to the oracle."""
    print("case: weighted split loop burst 100k x 1000, 30 ticks", flush=True)
    doc = weighted(100_000, 30)
    doc["instance"]["populations"][0]["initial_state"]["v"] = hex_array(np.full(100_000, -0.0495), "f32")
    protocol.seal(doc)
    expected = oracle.run(doc, lift_recording_budget=True)
    assert expected.synaptic_events >= 100_000 * 1000
    monkeypatch.setenv("ATLAS_HIP_PERSISTENT", "1")
    with HipExecutor(doc, device=0, lift_recording_budget=True, shape=WEIGHTED_SHAPE) as ex:
        assert ex.launch_mode == "persistent"
        result = ex.run()
        assert ex.launch_mode == "per-tick"
        dump, events = write_results(ex.document, result), write_events(ex.document, result)
    assert dump == expected.results and events == expected.events


def test_weighted_full_size_split_loop_equals_per_tick(monkeypatch):
    """The weighted network at its full size (1M neurons, 1e9 synapses with their own weights), 60
    ticks: the split loop's edge lists and one launch per tick give the same dump."""
    print("case: weighted split loop 1M x 1000, 60 ticks", flush=True)
    doc = weighted(1_000_000, 60)
    dump, events, result = run(doc, "persistent", monkeypatch, lift_recording_budget=True, verify_envelope=False)
    assert len(result["populations"][0]["spike_ticks"]) > 10_000
    tick_dump, tick_events, _ = run(doc, "per-tick", monkeypatch, lift_recording_budget=True, verify_envelope=False)
    assert tick_dump == dump and tick_events == events
