"""GPU parity: the HIP engine (through libatlas_sim_hip.so) against the reference's
golden dump and the CPU oracle, on the same AtlasIR documents.

Bar: spike rasters, counts, last-spike lists, refractory state and synaptic event
counts bit-exact; states bit-exact (both paths evaluate f64 registers with f32
storage rounding per statement, so the results are identical, not merely close).
"""
import numpy as np
import pytest

from atlas_hip import models
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
