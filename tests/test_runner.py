"""atlas-hip-runner argv and output conventions (model.rs:4596-4677, main.rs:2-7) without a GPU."""
import json

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
