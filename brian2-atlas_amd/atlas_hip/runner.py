"""``atlas-hip-runner``: the ``b2-runner`` command line on the MI355X engine.

Same argv, outputs and exit convention as the reference runner (run_cli,
brian2-rust/src/model.rs:4596-4677; main.rs:2-7):

    python -m atlas_hip.runner MODEL.json OUTPUT_DIRECTORY
    python -m atlas_hip.runner --validate MODEL.json
    python -m atlas_hip.runner --canonical-hashes MODEL.json

The reference's opt-in process budgets (``B2_MAX_IR_BYTES``, ``B2_MAX_NEURONS``, ...;
resource_limits.rs) are read and enforced before any device work (``limits``).

A run writes ``results.bin`` (B2DMP001 v3), ``events.bin`` (B2EVT001, when the
model has event streams) and ``summary.json`` (schema ``b2-result-dump-v3``)
into a new directory.  Errors print ``atlas-hip-runner: {error}`` on stderr and
exit with status 1.  ``--validate`` additionally proves that the HIP engine can
lower the model (it raises for constructs outside the supported subset).
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

from . import engine, limits, protocol
from .results import summary, write_events, write_results, write_summary_json

USAGE = ("usage: atlas-hip-runner MODEL.json OUTPUT_DIRECTORY | atlas-hip-runner --validate MODEL.json | "
         "atlas-hip-runner --canonical-hashes MODEL.json")


def _load(path: Path, ir_bytes: int) -> dict:
    """The document, refused beyond the IR byte budget before it is parsed (model.rs:4605-4658)."""
    if path.stat().st_size > ir_bytes:
        raise ValueError("IR exceeds the configured byte budget")
    return protocol.load(path)


def run(argv: list[str]) -> None:
    if len(argv) != 2:
        raise ValueError(USAGE)
    option, path = argv
    ir_bytes = limits.check_runner_environment()
    if option == "--canonical-hashes":
        document = _load(Path(path), ir_bytes)
        print(json.dumps(protocol.expected_protocol(document)["layers"], sort_keys=True, separators=(",", ":")))
        return
    if option == "--validate":
        document = _load(Path(path), ir_bytes)
        limits.check_document(document)
        engine.lower(document, verify_envelope=False)
        print("validated AtlasIR")
        return
    if option.startswith("--"):
        raise ValueError("unknown atlas-hip-runner option")
    model, directory = Path(option), Path(path)
    if directory.exists():
        raise ValueError("output directory already exists; choose a new directory")
    from .executor import HipExecutor
    document = _load(model, ir_bytes)
    limits.check_document(document)
    with HipExecutor(document) as executor:
        result = executor.run()
        document = executor.document
    started = time.perf_counter()
    results_bytes = write_results(document, result)
    events_bytes = write_events(document, result)
    directory.mkdir(parents=True)
    (directory / "results.bin").write_bytes(results_bytes)
    if events_bytes is not None:
        (directory / "events.bin").write_bytes(events_bytes)
    result["dump_write_seconds"] = time.perf_counter() - started
    write_summary_json(directory / "summary.json", summary(document, result, results_bytes, events_bytes))


def main(argv: list[str] | None = None) -> int:
    try:
        run(list(sys.argv[1:] if argv is None else argv))
    except Exception as error:  # the reference prints every error the same way
        print(f"atlas-hip-runner: {error}", file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
