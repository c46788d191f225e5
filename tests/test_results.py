"""B2DMP001 v3 / B2EVT001 writers and reader against the reference's own dump files."""
import json
import struct

import numpy as np
import pytest

from atlas_hip import results


def _result_from_dump(document, dump, events_bytes):
    """Rebuild an executor result dictionary from a parsed dump (the inverse of write_results)."""
    d = document["definition"]
    streams = _read_events(events_bytes)
    pops = []
    stream_index = 0
    for pdef, pd in zip(d["populations"], dump.populations):
        event_streams = {}
        for event in pdef["events"]:
            event_streams[event] = streams[stream_index]
            stream_index += 1
        pops.append({
            "states": {s["name"]: pd.states[k] for k, s in enumerate(pdef["states"])},
            "trace": {name: pd.samples[k] for k, name in enumerate(pdef["monitor"]["variables"])},
            "spike_ticks": pd.spikes[:, 0], "indices": pd.spikes[:, 1], "counts": pd.counts,
            "last_spikes": pd.last_fired,
            "refractory": None if pd.lastspike is None else {"lastspike": pd.lastspike,
                                                              "not_refractory": pd.not_refractory},
            "event_streams": event_streams})
    syns = [{"states": {s["name"]: sd["states"][k] for k, s in enumerate(sdef["states"])},
             "events": sd["delivered"], "edges": sd["edges"]} for sdef, sd in zip(d["synapses"], dump.synapses)]
    return {"populations": pops, "synapses": syns}


def _read_events(data):
    assert data[:8] == b"B2EVT001" and data[-8:] == b"B2EEND01"
    (count,) = struct.unpack_from("<Q", data, 8)
    offset, streams = 16, []
    for _ in range(count):
        (n,) = struct.unpack_from("<Q", data, offset)
        pairs = np.frombuffer(data, "<i8", 2 * n, offset + 8).reshape(n, 2)
        streams.append({"ticks": pairs[:, 0], "indices": pairs[:, 1]})
        offset += 8 + 16 * n
    return streams


def test_reference_dump_round_trip(golden):
    document = json.loads((golden / "reference_v1_model.json").read_text())
    data = (golden / "reference_v1_results.bin").read_bytes()
    events = (golden / "reference_v1_events.bin").read_bytes()
    dump = results.read_results(data, document)
    assert [p.count for p in dump.populations] == [80, 20]
    assert [len(p.spikes) for p in dump.populations] == [95, 60]
    assert [s["delivered"] for s in dump.synapses] == [505, 253, 423, 57]
    result = _result_from_dump(document, dump, events)
    assert results.write_results(document, result) == data
    assert results.write_events(document, result) == events


def test_summary_fields(golden):
    document = json.loads((golden / "reference_v1_model.json").read_text())
    data = (golden / "reference_v1_results.bin").read_bytes()
    events = (golden / "reference_v1_events.bin").read_bytes()
    result = _result_from_dump(document, results.read_results(data, document), events)
    result.update(timings=[{"input_seconds": 0.1, "command_seconds": 0.5, "gpu_seconds": 0.4,
                            "readback_seconds": 0.0}], numeric_profile="x", device="y", rng_profile=None)
    summary = results.summary(document, result, data, events)
    reference = json.loads((golden / "reference_v1_summary.json").read_text())
    for key in ("dump_bytes", "event_dump_bytes", "final_time_seconds", "neuron_count", "population_count",
                "schema", "spike_count", "synaptic_events"):
        assert summary[key] == reference[key], key


def test_truncated_dump_is_rejected(golden):
    document = json.loads((golden / "reference_v1_model.json").read_text())
    data = (golden / "reference_v1_results.bin").read_bytes()
    for bad in (data[:-1], b"B2DMP002" + data[8:]):
        try:
            results.read_results(bad, document)
        except ValueError:
            continue
        raise AssertionError("malformed dump accepted")


def _executor_shaped(document, data, events):
    """A result with every key HipExecutor.run() returns, rebuilt from a reference dump."""
    result = _result_from_dump(document, results.read_results(data, document), events)
    for pop in result["populations"]:
        pop["event_monitors"] = {}
    result.update(timings=[{"input_seconds": 0.01, "command_seconds": 0.25, "gpu_seconds": 0.2,
                            "readback_seconds": 0.02}],
                  numeric_profile="reference-f64-registers/f32-storage-hip-v1", device="test device",
                  run_seconds=0.3, compile_seconds=0.5, plan_sha256="0" * 64, rng_profile=None,
                  hip_runtime={"device_seconds": 0.2, "launches": 256})
    return result


def test_reference_writer_accepts_the_executor_contract(golden, tmp_path):
    """The INTEGRATION binding: the reference writer (metal.py:926-1014, restated in
    tests/reference_writer.py) consumes a HipExecutor-shaped result and writes the same
    results.bin / events.bin bytes as atlas_hip.results; its summary sums the timings list."""
    import reference_writer
    document = json.loads((golden / "reference_v1_model.json").read_text())
    data = (golden / "reference_v1_results.bin").read_bytes()
    events = (golden / "reference_v1_events.bin").read_bytes()
    result = _executor_shaped(document, data, events)
    summary = reference_writer.write_gpu_results(document, result, tmp_path / "out", engine="hip",
                                                 numeric_profile=result["numeric_profile"])
    assert (tmp_path / "out" / "results.bin").read_bytes() == data == results.write_results(document, result)
    assert (tmp_path / "out" / "events.bin").read_bytes() == events == results.write_events(document, result)
    assert summary["spike_count"] == 155 and summary["synaptic_events"] == 1238
    assert summary["timings"]["simulation_and_recording_seconds"] == 0.25
    assert summary["hip_timings"] == result["timings"]


def test_reference_writer_profile_checks(golden, tmp_path):
    """The consumer's checks: rng_profile must be None without random draws, and a model with
    draws demands the reference GPU's float32 profile, which the HIP engine does not claim (it
    draws the CPU engine's f64 counter values): the INTEGRATION binding changes that check."""
    import copy

    import reference_writer
    from atlas_hip import models
    document = json.loads((golden / "reference_v1_model.json").read_text())
    data = (golden / "reference_v1_results.bin").read_bytes()
    events = (golden / "reference_v1_events.bin").read_bytes()
    result = _executor_shaped(document, data, events)
    with pytest.raises(reference_writer.ConsumerRejected):
        reference_writer.write_gpu_results(document, dict(result, rng_profile="splitmix64-counter-v1"),
                                           tmp_path / "a", engine="hip", numeric_profile=result["numeric_profile"])
    random_doc = copy.deepcopy(models.poisson_network(20, 30, indegree=5, steps=5))
    from atlas_hip.executor import has_random
    assert has_random(random_doc["definition"]) and not has_random(document["definition"])
