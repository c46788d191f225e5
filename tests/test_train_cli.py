"""``atlas-hip-train`` (the ``b2-train`` CLI, train_main.rs:1-69): argv, request/result JSON,
error convention; the GPU case compares the CLI's result with the trainer called directly."""
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

from atlas_hip import train_cli, training

ROOT = Path(__file__).resolve().parents[1]


def _cli(*args, env=None):
    environment = dict(os.environ, PYTHONPATH=str(ROOT / "brian2-atlas_amd"), **(env or {}))
    return subprocess.run([sys.executable, "-m", "atlas_hip.train_cli", *map(str, args)], capture_output=True,
                          text=True, env=environment, timeout=300)


def test_usage_and_error_result(tmp_path):
    """Wrong argv and a bad request exit 1 with ``atlas-hip-train: message``; with
    B2_TRAIN_ERROR_RESULT=1 the message is written as b2-native-training-error-v1."""
    done = _cli(tmp_path / "only-one")
    assert done.returncode == 1 and done.stderr.strip() == f"atlas-hip-train: {train_cli.USAGE}"
    request = tmp_path / "request.json"
    request.write_text(json.dumps({"plan": {}, "operation": "train", "inputs": [], "labels": [], "bogus": 1}))
    result = tmp_path / "result.json"
    done = _cli(request, result, env={"B2_TRAIN_ERROR_RESULT": "1"})
    assert done.returncode == 1 and "unknown training request field 'bogus'" in done.stderr
    assert json.loads(result.read_text()) == {"schema": "b2-native-training-error-v1",
                                              "message": "unknown training request field 'bogus'"}


def test_request_size_limit(tmp_path):
    request = tmp_path / "big.json"
    with request.open("wb") as stream:
        stream.truncate(64 * 1024 * 1024 + 1)
    assert train_cli.main([str(request), str(tmp_path / "out.json")]) == 1


@pytest.mark.gpu
def test_cli_equals_the_trainer(tmp_path):
    """A train request through the CLI gives the trainer's own loss, gradients and state."""
    plan = training.lif_training_plan([8, 16, 4], backend="hip")
    rng = np.random.default_rng(3)
    inputs = (rng.random((5, 12, 8)) < 0.3).astype(float)
    labels = [0, 1, 2, 3, 1]
    trainer = training.NativeLIFTrainer(plan)
    state = json.loads(json.dumps(trainer.state))
    expected = trainer.step(inputs, labels)
    request = tmp_path / "request.json"
    request.write_text(json.dumps({"plan": plan, "state": state, "operation": "train", "inputs": inputs.tolist(),
                                   "labels": labels, "initial": None}))
    print("train cli", flush=True)
    done = _cli(request, tmp_path / "result.json")
    assert done.returncode == 0, done.stderr
    result = json.loads((tmp_path / "result.json").read_text())
    assert result["schema"] == "b2-lif-training-result-v1" and result["loss"] == expected["loss"]
    assert result["gradients"] == [list(g) for g in expected["gradients"]]
    assert result["state"] == json.loads(json.dumps(expected["state"]))
    assert np.array_equal(np.asarray(result["spikes"]).reshape(-1), np.asarray(expected["spikes"]).reshape(-1))
