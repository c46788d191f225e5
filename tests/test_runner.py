"""atlas-hip-runner argv and output conventions (model.rs:4596-4677, main.rs:2-7) without a GPU."""
import json

import pytest

from atlas_hip import runner


def test_canonical_hashes(golden, capsys):
    assert runner.main(["--canonical-hashes", str(golden / "atlasir_v1_minimal.json")]) == 0
    layers = json.loads(capsys.readouterr().out)
    assert layers == json.loads((golden / "atlasir_v1_hashes.json").read_text())["layers"]


def test_validate_lowers_the_model(golden, capsys):
    assert runner.main(["--validate", str(golden / "reference_v1_model.json")]) == 0
    assert capsys.readouterr().out.strip() == "validated AtlasIR"


def test_errors_print_prefixed_and_exit_1(golden, tmp_path, capsys):
    assert runner.main([]) == 1
    assert capsys.readouterr().err.startswith("atlas-hip-runner: usage:")
    assert runner.main(["--bogus", "x"]) == 1
    assert "unknown atlas-hip-runner option" in capsys.readouterr().err
    assert runner.main([str(golden / "reference_v1_model.json"), str(tmp_path)]) == 1
    assert "output directory already exists" in capsys.readouterr().err
    bad = tmp_path / "bad.json"
    doc = json.loads((golden / "reference_v1_model.json").read_text())
    doc["run"]["clocks"][0]["steps"] += 1
    bad.write_text(json.dumps(doc))
    assert runner.main(["--validate", str(bad)]) == 1
    assert "hash mismatch" in capsys.readouterr().err


def test_resource_budgets(tmp_path, monkeypatch, golden):
    """The reference's opt-in budgets (resource_limits.rs): malformed values are refused with its
    message, and a model beyond a budget is refused before any device work, through the CLI's
    error convention."""
    from atlas_hip import limits, models
    model = golden / "reference_v1_model.json"
    for bad in ["", "0", "-1", "+1", "1.5", " 1", "\uff11", "16000001"]:
        monkeypatch.setenv("B2_MAX_NEURONS", bad)
        with pytest.raises(limits.BudgetError, match="B2_MAX_NEURONS requires decimal digits in 1..16000000"):
            limits.check_runner_environment()
    monkeypatch.setenv("B2_MAX_NEURONS", "16000000")
    limits.check_runner_environment()
    monkeypatch.delenv("B2_MAX_NEURONS")
    document = json.loads(model.read_text())
    limits.check_document(document)
    cases = [("B2_MAX_NEURONS", "3", "invalid neuron count"), ("B2_MAX_STATEMENTS", "1", "too many statements"),
             ("B2_MAX_POPULATION_STATES", "1", "population state arrays"),
             ("B2_MAX_INITIAL_VALUES", "10", "probe array budget exceeded"),
             ("B2_MAX_POPULATION_STEPS", "2", "probe population duration budget exceeded")]
    for name, value, message in cases:
        monkeypatch.setenv(name, value)
        with pytest.raises(limits.BudgetError, match=message):
            limits.check_document(document)
        monkeypatch.delenv(name)
    doc = models.cuba_network(1000, steps=10)
    monkeypatch.setenv("B2_MAX_EXPLICIT_SYNAPSES", "100")
    with pytest.raises(limits.BudgetError, match="explicit synapse budget"):
        limits.check_document(doc)
    monkeypatch.delenv("B2_MAX_EXPLICIT_SYNAPSES")
    monkeypatch.setenv("B2_MAX_IR_BYTES", "1000")
    assert runner.main([str(model), str(tmp_path / "out")]) == 1
    assert not (tmp_path / "out").exists()
    assert runner.main(["--validate", str(model)]) == 1
