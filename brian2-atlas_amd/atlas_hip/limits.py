"""Opt-in process budgets of the runner (brian2-rust/src/resource_limits.rs:1-61; enforced by
run_cli and Model::validate, model.rs:1904, 2154, 2532, 3328-3482, 4592-4608).

Each budget is an environment variable holding decimal digits in 1..ceiling; unset means the
default.  The runner refuses a model that exceeds one before any device work."""
from __future__ import annotations

import os

# name: (default, ceiling)
BUDGETS = {
    "B2_MAX_INITIAL_VALUES": (100_000_000, 8_000_000_000),
    "B2_MAX_EXPLICIT_SYNAPSES": (50_000_000, 1_000_000_000),
    "B2_MAX_TIMED_ARRAY_VALUES": (10_000_000, 1_000_000_000),
    "B2_MAX_IR_BYTES": (2048 * 1_048_576, 64 * 1_073_741_824),
    "B2_MAX_NEURONS": (1_000_000, 16_000_000),
    "B2_MAX_POPULATION_STEPS": (10_000_000, 10_000_000),
    "B2_MAX_POPULATION_STATES": (32, 1024),
    "B2_MAX_POPULATION_PARAMETERS": (128, 1024),
    "B2_MAX_STATEMENTS": (128, 1024),
    "B2_MAX_SCRATCH_VALUES": (4_000_000, 128_000_000),
}


class BudgetError(ValueError):
    """A malformed budget variable or a model beyond a budget (the reference's messages)."""


def budget(name: str) -> int:
    """The budget's value: the variable's decimal digits (no sign, space or other digits), within
    1..ceiling, else the default when unset (resource_limits.rs:4-24)."""
    default, ceiling = BUDGETS[name]
    text = os.environ.get(name)
    if text is None:
        return default
    if not text or not all("0" <= c <= "9" for c in text) or not 1 <= int(text) <= ceiling:
        raise BudgetError(f"{name} requires decimal digits in 1..{ceiling}")
    return int(text)


def check_runner_environment() -> int:
    """The budgets run_cli reads before loading a model (model.rs:4605-4608); returns the IR byte
    budget."""
    ir_bytes = budget("B2_MAX_IR_BYTES")
    for name in ("B2_MAX_INITIAL_VALUES", "B2_MAX_NEURONS", "B2_MAX_POPULATION_STEPS"):
        budget(name)
    return ir_bytes


def _length(value) -> int:
    return 0 if value is None else (1 if isinstance(value, (str, int, float, bool)) else len(value))


def check_document(document: dict) -> None:
    """The model budgets Model::validate applies: neuron count, population steps and duration,
    states and parameters per population, statements per code object, explicit synapses, and
    the sum of every initial array's length (the probe array budget)."""
    d, inst = document["definition"], document["instance"]
    neurons = sum(int(p["count"]) for p in d["populations"])
    if not 1 <= neurons <= budget("B2_MAX_NEURONS"):
        raise BudgetError("invalid neuron count")
    steps_budget = budget("B2_MAX_POPULATION_STEPS")
    values = 0
    for pdef, pin in zip(d["populations"], inst["populations"]):
        if int(pdef["steps"]) > steps_budget or int(pdef["count"]) * int(pdef["steps"]) > 250_000_000_000:
            raise BudgetError("probe population duration budget exceeded")
        if len(pdef["states"]) > budget("B2_MAX_POPULATION_STATES"):
            raise BudgetError("population state arrays do not match definition")
        if len(pdef["parameters"]) > budget("B2_MAX_POPULATION_PARAMETERS"):
            raise BudgetError("population parameter arrays do not match definition")
        values += sum(_length(v) for v in pin["initial_state"].values())
        values += sum(_length(v) for v in pin["parameters"].values())
        refractory = pin.get("refractory") or {}
        values += _length(refractory.get("initial_lastspike")) + _length(refractory.get("initial_not_refractory"))
    statements = budget("B2_MAX_STATEMENTS")
    codes = [c for p in d["populations"] for c in p["code_objects"]] + \
        [c for s in d["synapses"] for c in s["code_objects"]]
    if any(len(c.get("scalar", [])) + len(c.get("vector", [])) > statements for c in codes):
        raise BudgetError("too many statements")
    explicit = budget("B2_MAX_EXPLICIT_SYNAPSES")
    for sin in inst["synapses"]:
        if sin["topology"]["kind"] == "explicit":
            if _length(sin["source"]) > explicit:
                raise BudgetError("explicit synapse budget exceeded")
            values += _length(sin["source"]) + _length(sin["target"])
        values += sum(_length(v) for v in sin.get("initial_state", {}).values())
        values += sum(_length(v) for v in sin.get("parameters", {}).values())
        values += sum(_length(pw.get("delay_ticks")) for pw in sin["pathways"])
    if values > budget("B2_MAX_INITIAL_VALUES"):
        raise BudgetError("probe array budget exceeded")
