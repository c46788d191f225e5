"""AtlasIR v1 integrity envelope against the reference's golden vectors
(brian2-rust/tests/golden/atlasir-v1 and b2ir-v1; model.rs:4596-4790)."""
import copy
import json

import pytest

from atlas_hip import protocol


@pytest.fixture(scope="module")
def minimal(golden):
    return json.loads((golden / "atlasir_v1_minimal.json").read_text())


@pytest.fixture(scope="module")
def legacy(golden):
    return json.loads((golden / "b2ir_v1_minimal.json").read_text())


def test_layer_and_document_hashes(golden, minimal):
    hashes = json.loads((golden / "atlasir_v1_hashes.json").read_text())
    assert protocol.layer_hashes(minimal) == hashes["layers"]
    assert protocol.document_sha256(minimal) == hashes["canonical_document_sha256"]
    assert minimal["protocol"]["layers"] == hashes["layers"]


def test_legacy_hashes_and_migration(golden, legacy, minimal):
    hashes = json.loads((golden / "b2ir_v1_hashes.json").read_text())
    assert protocol.layer_hashes(legacy) == hashes["layers"]
    assert protocol.document_sha256(legacy) == hashes["canonical_document_sha256"]
    migrated = protocol.load(legacy)
    assert migrated["schema"] == "atlasir-v1"
    assert migrated == minimal
    assert legacy["schema"] == "b2ir-v1"          # the input is not mutated


def test_load_accepts_paths_text_and_dicts(golden, minimal):
    path = golden / "atlasir_v1_minimal.json"
    assert protocol.load(path) == minimal
    assert protocol.load(path.read_text()) == minimal
    assert protocol.load(path.read_bytes()) == minimal


@pytest.mark.parametrize("layer", ["definition", "instance", "run"])
def test_tampered_layer_is_rejected(minimal, layer):
    doc = copy.deepcopy(minimal)
    doc[layer]["_tamper"] = 1
    with pytest.raises(protocol.ProtocolError, match="hash mismatch"):
        protocol.load(doc)
    protocol.load(doc, verify_envelope=False)


def test_malformed_documents_are_rejected(minimal):
    doc = copy.deepcopy(minimal)
    doc["schema"] = "atlasir-v2"
    with pytest.raises(protocol.ProtocolError, match="unsupported"):
        protocol.load(doc)
    doc = copy.deepcopy(minimal)
    doc["extra"] = {}
    with pytest.raises(protocol.ProtocolError, match="unknown"):
        protocol.load(doc)
    doc = copy.deepcopy(minimal)
    del doc["run"]
    with pytest.raises(protocol.ProtocolError, match="missing"):
        protocol.expected_protocol(doc)


def test_canonical_encoding_rules():
    assert protocol.canonical_bytes({"b": 1, "a": [1.5, "é"]}) == '{"a":[1.5,"é"],"b":1}'.encode()
    assert protocol.canonical_bytes(1e-7) == b"1e-07"
    assert protocol.canonical_bytes(1e16) == b"1e+16"
    assert protocol.canonical_bytes(0.1) == b"0.1"
    with pytest.raises(ValueError):
        protocol.canonical_bytes(float("nan"))
