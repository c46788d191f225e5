"""``atlas-hip-train``: the ``b2-train`` command line on the MI355X trainer.

Same argv, request and result JSON and exit convention as the reference's native
training CLI (brian2-rust/src/train_main.rs:1-69, request and result schemas
training.rs:150-208) for the plans the HIP trainer runs (dense layered
``b2-lif-training-plan-v1`` and projection-graph ``b2-lif-training-plan-v2``):

    python -m atlas_hip.train_cli REQUEST.json RESULT.json

The request holds ``plan``, ``state`` (weights, Adam moments and step; null for the
plan's initial weights), ``operation`` (train, gradients or evaluate), ``inputs``
(batch x time x input), ``labels`` and ``initial`` (per-sample initial membranes, or
null).  The result is ``b2-lif-training-result-v1``.  Requests over 64 MiB are refused.
Errors print ``atlas-hip-train: {message}`` on stderr and exit with status 1; with
``B2_TRAIN_ERROR_RESULT=1`` the message is also written to RESULT.json as
``b2-native-training-error-v1`` (through a temporary file and a rename).
"""
from __future__ import annotations

import json
import os
import sys
from pathlib import Path

import numpy as np

USAGE = "usage: atlas-hip-train REQUEST.json RESULT.json"
REQUEST_LIMIT = 64 * 1024 * 1024
REQUEST_KEYS = {"plan", "state", "operation", "inputs", "labels", "initial"}


def _plain(value):
    if isinstance(value, np.ndarray):
        return value.tolist()
    if isinstance(value, dict):
        return {k: _plain(v) for k, v in value.items()}
    if isinstance(value, (list, tuple)):
        return [_plain(v) for v in value]
    if isinstance(value, np.generic):
        return value.item()
    return value


def execute(request: dict) -> dict:
    """Run one training request (training.rs execute for a dense v1 or projection-graph v2 plan)."""
    from .training import NativeLIFTrainer
    unknown = set(request) - REQUEST_KEYS
    if unknown:
        raise ValueError(f"unknown training request field {sorted(unknown)[0]!r}")
    plan, state = request["plan"], request.get("state")
    trainer = NativeLIFTrainer(plan, weights=None if state is None else state["weights"])
    if state is not None:
        counts = [len(w) for w in trainer.state["weights"]]
        if ([len(m) for m in state["first_moment"]] != counts or [len(m) for m in state["second_moment"]] != counts
                or int(state["step"]) < 0):
            raise ValueError("training state does not match the plan")
        trainer.state.update(first_moment=[list(map(float, m)) for m in state["first_moment"]],
                             second_moment=[list(map(float, m)) for m in state["second_moment"]],
                             step=int(state["step"]))
    inputs = np.asarray(request["inputs"], np.float64)
    out = trainer.execute(inputs, request["labels"], operation=request["operation"], initial=request.get("initial"))
    batch, time = inputs.shape[:2]
    neurons = sum(plan["sizes"][1:])
    out.update(gpu_dispatches=1, tape_bytes=int(batch * time * neurons * 4 * 3),
               spikes=np.asarray(out["spikes"]).reshape(batch, time, -1),
               final_membrane=np.asarray(out["final_membrane"]).reshape(batch, -1),
               initial_gradients=np.asarray(out["initial_gradients"]).reshape(batch, -1),
               logits=np.asarray(out["logits"]).reshape(batch, -1))
    out.pop("losses", None)
    return _plain(out)


def _write_error(output: str, message: str) -> None:
    target = Path(output)
    temporary = target.with_suffix(".error-0.tmp")
    try:
        temporary.write_text(json.dumps({"schema": "b2-native-training-error-v1", "message": message}))
        os.replace(temporary, target)
    except OSError:
        pass


def main(argv: list[str] | None = None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    try:
        if len(argv) != 2:
            raise ValueError(USAGE)
        request_path, result_path = argv
        if Path(request_path).stat().st_size > REQUEST_LIMIT:
            raise ValueError("training request exceeds 64 MiB input limit")
        request = json.loads(Path(request_path).read_bytes())
        result = execute(request)
        Path(result_path).write_text(json.dumps(result))
        return 0
    except Exception as error:  # the reference reports every failure the same way
        message = str(error) or type(error).__name__
        if len(message) > 4096:
            message = message[:4096 - len(" [truncated]")] + " [truncated]"
        if os.environ.get("B2_TRAIN_ERROR_RESULT") == "1" and len(argv) == 2:
            _write_error(argv[1], message)
        print(f"atlas-hip-train: {message}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    sys.exit(main())
