"""AtlasIR v1 integrity envelope: canonical JSON, layer hashes, legacy migration.

Restates the reader side of the frozen protocol:

* canonical encoding ``atlasir-canonical-json-v1`` (AtlasIR.md section 3): sorted
  keys, compact separators, UTF-8, shortest round-trip float digits;
* layer hashes ``sha256(canonical(definition|instance|run))`` and the envelope
  check of ``b2-runner`` (``run_cli`` / ``expected_protocol`` model.rs:4596-4736);
* migration of the legacy ``b2ir-v1`` envelope: verify it first, then relabel the
  schema and rebuild the envelope (``prepare_protocol`` model.rs:4738-4790).

Python's ``json`` float formatting is ``repr``: shortest round-trip digits, fixed
notation for decimal exponents -4..15, otherwise ``e`` with a sign and at least
two digits, which is exactly the number format the canonical encoding fixes.
"""
from __future__ import annotations

import copy
import hashlib
import json
from pathlib import Path

CURRENT_SCHEMA = "atlasir-v1"
LEGACY_SCHEMA = "b2ir-v1"
_IDENTIFIERS = {
    CURRENT_SCHEMA: ("atlasir", "atlasir-canonical-json-v1"),
    LEGACY_SCHEMA: ("b2ir", "b2ir-canonical-json-v1"),
}


class ProtocolError(ValueError):
    """The document is not a verifiable AtlasIR v1 document."""


def canonical_bytes(value) -> bytes:
    return json.dumps(value, sort_keys=True, separators=(",", ":"), ensure_ascii=False,
                      allow_nan=False).encode("utf-8")


def sha256_hex(value) -> str:
    return hashlib.sha256(canonical_bytes(value)).hexdigest()


def layer_hashes(document: dict) -> dict:
    missing = [layer for layer in ("definition", "instance", "run") if layer not in document]
    if missing:
        raise ProtocolError(f"missing {missing[0]}")
    return {layer: sha256_hex(document[layer]) for layer in ("definition", "instance", "run")}


def expected_protocol(document: dict) -> dict:
    schema = document.get("schema")
    if schema not in _IDENTIFIERS:
        raise ProtocolError(f"unsupported AtlasIR schema {schema!r}")
    name, encoding = _IDENTIFIERS[schema]
    return {"name": name, "version": {"major": 1, "minor": 0}, "canonical_encoding": encoding,
            "hash_algorithm": "sha256", "layers": layer_hashes(document)}


def seal(document: dict) -> dict:
    """Attach (or replace) the integrity envelope of a document under construction."""
    document["protocol"] = expected_protocol(document)
    return document


def verify(document: dict) -> None:
    if document.get("protocol") != expected_protocol(document):
        raise ProtocolError("AtlasIR canonical layer hash mismatch")


def load(source, *, verify_envelope: bool = True) -> dict:
    """Read, verify and (for ``b2ir-v1``) migrate an AtlasIR document.

    ``source`` may be a path, a JSON string/bytes, or an already-parsed dict.
    The input dict is never mutated.
    """
    if isinstance(source, dict):
        document = copy.deepcopy(source)
    elif isinstance(source, (bytes, bytearray)):
        document = json.loads(source)
    elif isinstance(source, str) and source.lstrip().startswith("{"):
        document = json.loads(source)
    else:
        document = json.loads(Path(source).read_text())
    if not isinstance(document, dict):
        raise ProtocolError("AtlasIR root must be an object")
    extra = set(document) - {"schema", "protocol", "definition", "instance", "run"}
    if extra:
        raise ProtocolError(f"unknown AtlasIR root field {sorted(extra)[0]!r}")
    schema = document.get("schema")
    if schema not in _IDENTIFIERS:
        raise ProtocolError(f"unsupported AtlasIR schema {schema!r}")
    if verify_envelope:
        verify(document)
    if schema == LEGACY_SCHEMA:
        document["schema"] = CURRENT_SCHEMA
        seal(document)
    return document


def document_sha256(document: dict) -> str:
    return sha256_hex(document)
