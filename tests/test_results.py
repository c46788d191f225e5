"""B2DMP001 v3 / B2EVT001 writers and reader against the reference's own dump files."""
import json
import struct

import numpy as np

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
        streams.append((pairs[:, 0], pairs[:, 1]))
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
    result.update(timings={"simulation_seconds": 0.5}, numeric_profile="x", device="y")
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
