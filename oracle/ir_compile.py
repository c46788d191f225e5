"""CPU oracle front end: AtlasIR -> flat blob for the C interpreter (``atlas_oracle.c``).

TEST INFRASTRUCTURE ONLY.  Nothing in the product path may import this module;
only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg
use it, and only as the checker / the timed CPU baseline.

This file restates the *compile* half of the reference CPU engine
(``brian2-rust/src/executor.rs``) in Python:

* ``Program`` follows ``Program::compile`` / ``statements`` / ``expression``
  (executor.rs:5046-5486): SSA registers, one register per expression node,
  ``Select`` for conditional statements, scalar statements evaluated once per
  phase and broadcast (executor.rs:5093-5104), and writes bound through the
  code object's declared ``effects.writes`` (executor.rs:5105-5113).
* dtype inference follows ``Expr::infer`` (model.rs:1251-1531): it decides
  integer versus float opcodes and the source dtype of casts.
* population inputs follow ``population_runtime`` (executor.rs:1757-2111);
  synapse inputs follow ``Runtime::new`` (executor.rs:3507-3633).

The C side restates the execution half: ``Program::prepare/run/commit``,
``evaluate``, the schedule dispatch of ``Runtime::advance``, pathway queues,
monitors and the ``B2DMP001`` / ``B2EVT001`` dump writers.

Supported subset (anything else raises ``UnsupportedModel`` before running):
populations with state_update / threshold / reset / run_regularly /
subexpression_update code objects, fixed refractory, spike monitors, the
population state monitor; synapses with explicit, fixed_total or
fixed_indegree topology and pre/post pathways.  Linked variables, spatial or
adaptive integrators, summed variables, synapse state updates, event monitors,
spike generators and TimedArrays are rejected.
"""
from __future__ import annotations

import hashlib
import json
import math
import struct
from pathlib import Path

MAGIC = b"ATLORC01"

DTYPES = {"f32": 0, "f64": 1, "i32": 2, "i64": 3, "u32": 4, "u64": 5,
          "bool": 6, "index": 7, "tick": 8}
INTEGER = {"i32", "i64", "u32", "u64"}

# Input kinds (executor.rs:4827-4847).
IN_CONSTANT, IN_TIME, IN_INDEX, IN_STATE, IN_PRE, IN_POST, IN_SYN, IN_PARAM, \
    IN_LASTSPIKE, IN_AVAILABLE, IN_RANDOM, IN_NORMAL = range(12)
# Domains (executor.rs:330-336).
D_NEURON, D_PRE, D_POST, D_EDGE = range(4)
# Write targets (executor.rs:4861-4866).
W_NEURON, W_PRE, W_SYN, W_AVAILABLE = range(4)

# Opcodes: the order must match ``enum op`` in atlas_oracle.c.
OPS = ["neg", "not", "abs", "arccos", "arcsin", "arctan", "ceil", "cos", "cosh",
       "exp", "expm1", "exprel", "floor", "trunc", "round_f32", "cast",
       "int_unary", "int_binary", "timestep", "tick_offset", "log", "log10",
       "log1p", "sign", "sin", "sinh", "sqrt", "tan", "tanh", "add", "sub", "mul",
       "div", "pow", "mod", "floordiv", "eq", "ne", "gt", "ge", "lt", "le", "and",
       "or", "clip", "select", "binomial", "poisson"]
OP = {name: code for code, name in enumerate(OPS)}
INT_UNARY = {"neg": 0, "abs": 1}
INT_BINARY = {"add": 0, "sub": 1, "mul": 2, "mod": 3, "floordiv": 4,
              "gt": 5, "ge": 6, "lt": 7, "le": 8}
UNARY_MATH = {"arccos", "arcsin", "arctan", "ceil", "cos", "cosh", "exp", "expm1",
              "exprel", "floor", "trunc", "log", "log10", "log1p", "sign", "sin",
              "sinh", "sqrt", "tan", "tanh"}
BINARY = {"add", "sub", "mul", "div", "pow", "mod", "floordiv", "eq", "ne", "gt",
          "ge", "lt", "le", "and", "or"}
RELATIONAL = {"gt", "ge", "lt", "le"}

# Population code-object kinds understood by the C dispatcher.
POP_KINDS = {"subexpression_update": 0, "state_update": 1, "threshold": 2,
             "run_regularly": 3, "reset": 4}


class UnsupportedModel(ValueError):
    """The model is valid AtlasIR but outside the oracle's supported subset."""


def f64_bits(value: float) -> int:
    return struct.unpack("<Q", struct.pack("<d", value))[0]


def decode_f64(bits: str) -> float:
    return struct.unpack(">d", bytes.fromhex(bits))[0]


def decode_f32(bits: str) -> float:
    return struct.unpack(">f", bytes.fromhex(bits))[0]


def decode_typed(bits: str, dtype: str) -> float:
    """``decode_typed_float`` (model.rs:883-908): register value of an encoded scalar."""
    if dtype == "f32":
        return decode_f32(bits)
    if dtype == "f64":
        return decode_f64(bits)
    if dtype == "bool":
        return {"00": 0.0, "01": 1.0}[bits]
    # integers keep their raw two's-complement bits inside the f64 register
    return struct.unpack("<d", struct.pack("<Q", int(bits, 16)))[0]


def load_document(source) -> dict:
    if isinstance(source, dict):
        return source
    return json.loads(Path(source).read_text())


class Blob:
    def __init__(self) -> None:
        self.parts: list[bytes] = [MAGIC]

    def u(self, value: int) -> None:
        self.parts.append(struct.pack("<Q", value & 0xFFFFFFFFFFFFFFFF))

    def i(self, value: int) -> None:
        self.parts.append(struct.pack("<q", value))

    def f(self, value: float) -> None:
        self.parts.append(struct.pack("<d", value))

    def raw(self, data: bytes) -> None:
        self.u(len(data))
        self.parts.append(data)
        pad = (-len(data)) % 8
        if pad:
            self.parts.append(b"\0" * pad)

    def f64s(self, values) -> None:
        self.raw(struct.pack(f"<{len(values)}d", *values))

    def u64s(self, values) -> None:
        self.raw(struct.pack(f"<{len(values)}Q", *values))

    def bytes(self) -> bytes:
        return b"".join(self.parts)


def encode_state(blob: Blob, dtype: str, values: list[str]) -> None:
    """Storage-typed initial values of one SoA state (``StateArray::from_encoded``)."""
    blob.u(DTYPES[dtype])
    if dtype == "f32":
        data = b"".join(bytes.fromhex(v)[::-1] for v in values)
    elif dtype == "f64":
        data = b"".join(bytes.fromhex(v)[::-1] for v in values)
    elif dtype == "bool":
        data = bytes({"00": 0, "01": 1}[v] for v in values)
    elif dtype in ("i32", "u32"):
        data = b"".join(struct.pack("<I", int(v, 16)) for v in values)
    elif dtype in ("i64", "u64"):
        data = b"".join(struct.pack("<Q", int(v, 16)) for v in values)
    else:
        raise UnsupportedModel(f"unsupported state dtype {dtype}")
    blob.u(len(values))
    blob.raw(data)


class Program:
    """Restatement of ``Program::compile`` (executor.rs:5046-5113)."""

    def __init__(self, code: dict, inputs: dict, writable: dict, functions: dict):
        for statement in code["scalar"] + code["vector"]:
            if statement.get("condition") is not None and not isinstance(statement["condition"], str):
                raise UnsupportedModel("statement condition must be a symbol")
        if code.get("adaptive") is not None:
            raise UnsupportedModel("adaptive integrators are not supported")
        self.inputs = inputs
        self.functions = functions
        self.nreg = 0
        self.bindings: list[tuple[int, tuple]] = []
        self.symbols: dict[str, int] = {}
        self.symbol_dtypes = {name: inp[-1] for name, inp in inputs.items()}
        self.rng_domain = D_EDGE if code["iteration_domain"] in ("all_synapses", "active_synapses") else D_NEURON
        self.scalar = self.statements(code["scalar"])
        self.scalar_random = sorted(slot for slot, inp in self.bindings if inp[0] in (IN_RANDOM, IN_NORMAL))
        broadcast = list(range(self.nreg))
        self.vector = self.statements(code["vector"])
        broadcast += [slot for slot, inp in self.bindings if inp[0] in (IN_CONSTANT, IN_TIME)]
        self.broadcast = sorted(set(broadcast))
        self.writes = []
        for name in code["effects"]["writes"]:
            if name not in writable:
                raise UnsupportedModel(f"write to {name} is not a writable target")
            self.writes.append((writable[name], self.symbols[name]))
        self.condition = self.symbols["_cond"] if code["kind"] == "threshold" else -1

    # -- register allocation ---------------------------------------------------------
    def register(self) -> int:
        slot = self.nreg
        self.nreg += 1
        return slot

    def input(self, value: tuple) -> int:
        slot = self.register()
        self.bindings.append((slot, value))
        return slot

    def resolve(self, name: str) -> int:
        if name in self.symbols:
            return self.symbols[name]
        if name not in self.inputs:
            raise UnsupportedModel(f"missing plan input {name!r}")
        slot = self.input(self.inputs[name])
        self.symbols[name] = slot
        return slot

    # -- dtype inference (model.rs:1251-1531) ----------------------------------------
    def infer(self, expr: dict) -> str:
        op = expr["op"]
        if op == "literal":
            return "f64"
        if op == "boolean":
            return "bool"
        if op in ("integer", "cast"):
            return expr["dtype"]
        if op in ("rand", "randn", "binomial", "poisson", "timed_array", "bool_to_f64",
                  "index_to_f64", "tick_to_f64", "f32_to_f64", "div", "clip"):
            return "f64"
        if op == "f64_to_f32":
            return "f32"
        if op in ("timestep", "tick_offset"):
            return "tick"
        if op == "load":
            return self.symbol_dtypes[expr["name"]]
        if op == "call":
            return self.functions[expr["function"]]["return_dtype"]
        if op in ("neg", "abs"):
            return self.infer(expr["arg"])
        if op in ("not", "eq", "ne", "and", "or") or op in RELATIONAL:
            return "bool"
        if op in UNARY_MATH:
            return "f64"
        if op in ("add", "sub", "mul", "pow", "mod", "floordiv"):
            left = self.infer(expr["left"])
            right = self.infer(expr["right"])
            return left if left == right and left in INTEGER else "f64"
        raise UnsupportedModel(f"unsupported expression op {op!r}")

    # -- expression lowering (executor.rs:5151-5445) ---------------------------------
    def expression(self, expr: dict, guard: int, ops: list) -> int:
        op = expr["op"]
        third = -1
        param = 0
        if op == "literal":
            return self.input((IN_CONSTANT, decode_f64(expr["bits"]), "f64"))
        if op == "boolean":
            return self.input((IN_CONSTANT, 1.0 if expr["value"] else 0.0, "bool"))
        if op == "integer":
            dtype = expr["dtype"]
            value = int(expr["value"])
            raw = value & (0xFFFFFFFF if dtype in ("i32", "u32") else 0xFFFFFFFFFFFFFFFF)
            return self.input((IN_CONSTANT, struct.unpack("<d", struct.pack("<Q", raw))[0], dtype))
        if op == "rand":
            return self.input((IN_RANDOM, expr["stream"], self.rng_domain, "f64"))
        if op == "randn":
            return self.input((IN_NORMAL, expr["stream"], self.rng_domain, "f64"))
        if op == "load":
            return self.resolve(expr["name"])
        if op in ("bool_to_f64", "index_to_f64", "tick_to_f64", "f32_to_f64"):
            return self.expression(expr["arg"], guard, ops)
        if op == "call":
            return self.call(expr, guard, ops)
        if op == "cast":
            source = self.infer(expr["arg"])
            slot = self.expression(expr["arg"], guard, ops)
            code, left, right, param = OP["cast"], slot, slot, (DTYPES[source] << 8) | DTYPES[expr["dtype"]]
        elif op == "f64_to_f32":
            slot = self.expression(expr["arg"], guard, ops)
            code, left, right = OP["round_f32"], slot, slot
        elif op == "timestep":
            left = self.expression(expr["time"], guard, ops)
            right = self.expression(expr["dt"], guard, ops)
            code = OP["timestep"]
        elif op == "tick_offset":
            slot = self.expression(expr["tick"], guard, ops)
            code, left, right, param = OP["tick_offset"], slot, slot, int(expr["offset"])
        elif op == "binomial":
            slot = self.expression(expr["p"], guard, ops)
            code, left, right = OP["binomial"], slot, slot
            param = (expr["stream"], expr["n"], 1 if expr["approximate"] else 0, self.rng_domain)
        elif op == "poisson":
            slot = self.expression(expr["lambda"], guard, ops)
            code, left, right = OP["poisson"], slot, slot
            param = (expr["stream"], self.rng_domain)
        elif op in ("neg", "not", "abs") or op in UNARY_MATH:
            slot = self.expression(expr["arg"], guard, ops)
            dtype = self.infer(expr["arg"])
            if op in ("neg", "abs") and dtype in INTEGER:
                code, param = OP["int_unary"], (DTYPES[dtype] << 8) | INT_UNARY[op]
            else:
                code = OP[op]
            left = right = slot
        elif op in BINARY:
            dtype = self.infer(expr["left"])
            if dtype in INTEGER and op in INT_BINARY:
                code, param = OP["int_binary"], (DTYPES[dtype] << 8) | INT_BINARY[op]
            else:
                code = OP[op]
            left = self.expression(expr["left"], guard, ops)
            right = self.expression(expr["right"], guard, ops)
        elif op == "clip":
            left = self.expression(expr["value"], guard, ops)
            right = self.expression(expr["min"], guard, ops)
            third = self.expression(expr["max"], guard, ops)
            code = OP["clip"]
        else:
            raise UnsupportedModel(f"unsupported expression op {op!r}")
        output = self.register()
        ops.append((code, left, right, third, guard, output, param))
        return output

    def call(self, expr: dict, guard: int, ops: list) -> int:
        contract = self.functions.get(expr["function"])
        if contract is None or contract.get("body") is None:
            raise UnsupportedModel("native-only Function")
        slots = [self.expression(argument, guard, ops) for argument in expr["arguments"]]
        previous = []
        for argument, slot in zip(contract["arguments"], slots):
            previous.append((argument["name"], self.symbols.get(argument["name"]),
                             self.symbol_dtypes.get(argument["name"])))
            self.symbols[argument["name"]] = slot
            self.symbol_dtypes[argument["name"]] = argument["dtype"]
        result = self.expression(contract["body"], guard, ops)
        for name, slot, dtype in previous:
            if slot is None:
                self.symbols.pop(name, None)
            else:
                self.symbols[name] = slot
            if dtype is None:
                self.symbol_dtypes.pop(name, None)
            else:
                self.symbol_dtypes[name] = dtype
        return result

    def statements(self, statements: list) -> list:
        ops: list = []
        for statement in statements:
            condition = statement.get("condition")
            guard = self.resolve(condition) if condition is not None else -1
            old = -1
            if guard >= 0:
                target = statement["target"]
                if target in self.symbols:
                    old = self.symbols[target]
                elif target in self.inputs:
                    old = self.resolve(target)
            value = self.expression(statement["value"], guard, ops)
            if old >= 0:
                output = self.register()
                ops.append((OP["select"], value, old, -1, guard, output, 0))
                value = output
            self.symbols[statement["target"]] = value
            self.symbol_dtypes[statement["target"]] = statement["dtype"]
        return ops

    # -- serialisation ---------------------------------------------------------------
    def emit(self, blob: Blob, param_arrays: dict) -> None:
        blob.u(self.nreg)
        blob.u(len(self.bindings))
        for slot, inp in self.bindings:
            kind = inp[0]
            blob.u(slot)
            blob.u(kind)
            if kind == IN_CONSTANT:
                blob.f(inp[1])
                blob.u(DTYPES[inp[2]])
            elif kind == IN_INDEX:
                blob.u(inp[1])
            elif kind == IN_STATE:
                blob.u(inp[1]); blob.u(inp[2])
            elif kind in (IN_PRE, IN_POST, IN_SYN):
                blob.u(inp[1])
            elif kind == IN_PARAM:
                # (IN_PARAM, key, domain, dtype): values live in the owner's table
                blob.u(param_arrays[inp[1]]); blob.u(inp[2])
            elif kind == IN_AVAILABLE:
                blob.u(inp[1])
            elif kind in (IN_RANDOM, IN_NORMAL):
                blob.u(inp[1]); blob.u(inp[2])
        blob.u64s(self.scalar_random)
        blob.u64s(self.broadcast)
        for ops in (self.scalar, self.vector):
            blob.u(len(ops))
            for code, left, right, third, guard, output, param in ops:
                blob.u(code); blob.u(left); blob.u(right); blob.i(third); blob.i(guard); blob.u(output)
                if isinstance(param, tuple):
                    values = list(param) + [0] * (4 - len(param))
                else:
                    values = [param, 0, 0, 0]
                for value in values:
                    blob.i(value)
        blob.u(len(self.writes))
        for (kind, index), register in self.writes:
            blob.u(kind); blob.u(index); blob.u(register)
        blob.i(self.condition)


def _parameters(inputs: dict, symbols: list, values: dict, domain: int, owner: str,
                tables: list, generated: dict) -> None:
    """``add_parameters`` (executor.rs:6214-6244)."""
    for symbol in symbols:
        name = symbol["name"]
        if symbol["index_domain"] == "scalar":
            inputs[name] = (IN_CONSTANT, decode_typed(values[name][0], symbol["dtype"]), symbol["dtype"])
            continue
        key = (owner, name)
        if name in generated:
            tables.append((key, ("generated", generated[name])))
        else:
            tables.append((key, ("values", [decode_typed(v, symbol["dtype"]) for v in values[name]])))
        inputs[name] = (IN_PARAM, key, domain, symbol["dtype"])


def _initializer(blob: Blob, spec: dict, delay_dt: float | None = None) -> None:
    """Procedural initializer (model.rs:465-530); values are materialised in C.

    A delay initializer (``delay_dt`` given) clips a clipped normal to
    [max(minimum or 0, 0), maximum or dt * 1e6], as materialize_delay_initializer
    does (executor.rs:160-187); a uniform one is used as declared."""
    if spec["kind"] == "uniform":
        blob.u(0); blob.u(spec["stream"])
        blob.f(decode_f64(spec["minimum"])); blob.f(decode_f64(spec["maximum"]))
        blob.f(0.0); blob.f(0.0); blob.u(1); blob.u(1)
    elif spec["kind"] == "clipped_normal":
        low = decode_f64(spec["minimum"]) if spec.get("minimum") is not None else None
        high = decode_f64(spec["maximum"]) if spec.get("maximum") is not None else None
        if delay_dt is not None:
            low = max(0.0 if low is None else low, 0.0)
            high = delay_dt * 1_000_000.0 if high is None else high
        blob.u(1); blob.u(spec["stream"])
        blob.f(0.0 if low is None else low)
        blob.f(0.0 if high is None else high)
        blob.f(decode_f64(spec["mean"])); blob.f(decode_f64(spec["std"]))
        blob.u(0 if low is None else 1); blob.u(0 if high is None else 1)
    else:
        raise UnsupportedModel(f"unsupported initializer {spec['kind']!r}")


def _read_binary_csr(topo: dict, sources: int, targets: int):
    """read_binary_csr (binary_topology.rs:24-130): a B2CSR001 file's edges (source-major,
    file order) and columns, with the reference's checks."""
    edges, columns = int(topo["edge_count"]), int(topo["column_count"])
    if not (0 < sources <= 1_000_000 and 0 < targets <= 1_000_000 and 0 < edges <= 100_000_000 and columns <= 128):
        raise UnsupportedModel("invalid binary CSR shape")
    with open(topo["path"], "rb") as stream:
        data = stream.read()
    if len(data) != 40 + (sources + 1) * 8 + edges * (4 + 8 * columns):
        raise UnsupportedModel("binary CSR file length mismatch")
    if hashlib.sha256(data).hexdigest() != str(topo["sha256"]).lower():
        raise UnsupportedModel("binary CSR checksum mismatch")
    if data[:8] != b"B2CSR001" or struct.unpack_from("<4Q", data, 8) != (sources, targets, edges, columns):
        raise UnsupportedModel("binary CSR header mismatch")
    offsets = struct.unpack_from(f"<{sources + 1}Q", data, 40)
    if offsets[0] != 0:
        raise UnsupportedModel("binary CSR offsets must start at zero")
    source = []
    for neuron in range(sources):
        if not offsets[neuron] <= offsets[neuron + 1] <= edges:
            raise UnsupportedModel("invalid binary CSR offsets")
        source.extend([neuron] * (offsets[neuron + 1] - offsets[neuron]))
    if offsets[-1] != edges:
        raise UnsupportedModel("binary CSR final offset mismatch")
    at = 40 + (sources + 1) * 8
    target = list(struct.unpack_from(f"<{edges}I", data, at))
    if any(value >= targets for value in target):
        raise UnsupportedModel("binary CSR target outside population")
    at += 4 * edges
    values = [struct.unpack_from(f"<{edges}d", data, at + 8 * edges * c) for c in range(columns)]
    if any(not math.isfinite(v) for column in values for v in column):
        raise UnsupportedModel("nonfinite binary CSR parameter")
    return source, target, values


def compile_model(source, *, lift_recording_budget: bool = False) -> bytes:
    """Compile an AtlasIR document (path, JSON text path, or dict) into the oracle blob."""
    doc = load_document(source)
    if doc.get("schema") not in ("atlasir-v1", "b2ir-v1"):
        raise UnsupportedModel(f"unsupported schema {doc.get('schema')!r}")
    d = doc["definition"]
    inst = doc["instance"]
    run = doc["run"]
    functions = {f["name"]: f for f in d["functions"]}
    blob = Blob()
    blob.u(1 if lift_recording_budget else 0)
    blob.u(len(d["clocks"]))
    for clock, rclock in zip(d["clocks"], run["clocks"]):
        blob.f(decode_f64(clock["dt"])); blob.u(rclock["start_tick"]); blob.u(rclock["steps"])
    blob.f(decode_f64(run["start"])); blob.f(decode_f64(run["duration"]))
    blob.u(int(inst["rng_seed"])); blob.u(int(inst["neuron_count"]))

    # ---- populations -------------------------------------------------------------------
    blob.u(len(d["populations"]))
    for index, (pdef, pin) in enumerate(zip(d["populations"], inst["populations"])):
        if pdef.get("linked_variables"):
            raise UnsupportedModel("linked variables are not supported")
        if pdef.get("spatial"):
            raise UnsupportedModel("spatial neurons are not supported")
        # rate monitors are a layout over the spike monitor (model.rs:3379-3386): nothing to run
        rate_names = [m["name"] for m in pdef.get("rate_monitors", [])]
        if (len(set(rate_names)) != len(rate_names) or any(m["dtype"] not in ("f32", "f64") for m in pdef.get("rate_monitors", []))
                or (rate_names and pdef.get("spike_monitor") is None)):
            raise UnsupportedModel("invalid rate monitor layout")
        if pdef.get("monitor_expressions") or pdef.get("monitor_timed_arrays"):
            raise UnsupportedModel("monitor expressions are not supported")
        generator = pin.get("spike_generator")
        if generator is not None and (pdef["code_objects"] or pdef["states"]):
            raise UnsupportedModel("a spike generator population has no code objects or states")
        count = pdef["count"]
        dt = decode_f64(pdef["dt"])
        blob.u(count); blob.u(pdef["clock"]); blob.f(dt); blob.u(pdef["steps"])
        blob.u(pdef["monitor"]["window_steps"])
        blob.u(len(pdef["states"]))
        for symbol in pdef["states"]:
            encode_state(blob, symbol["dtype"], pin["initial_state"][symbol["name"]])
        refr = pin.get("refractory")
        if (refr is None) != (pdef.get("refractory") is None):
            raise UnsupportedModel("refractory definition/instance mismatch")
        if refr is not None:
            blob.u(1)
            blob.u(1 if pdef["refractory"]["mode"] == "fixed" else 0)
            blob.u(refr["period_ticks"])
            blob.f64s([decode_f64(v) for v in refr["initial_lastspike"]])
            blob.raw(bytes(1 if v else 0 for v in refr["initial_not_refractory"]))
        else:
            blob.u(0)
        events = pdef["events"]
        blob.u(len(events))
        blob.i(events.index("spike") if "spike" in events else -1)
        # SpikeGeneratorGroup schedule (model.rs:3762-3790 checks it)
        gen_ticks = [int(v) for v in generator["spike_ticks"]] if generator else []
        gen_neurons = [int(v) for v in generator["spike_indices"]] if generator else []
        if generator is not None:
            start, steps = run["clocks"][pdef["clock"]]["start_tick"], pdef["steps"]
            pairs = list(zip(gen_ticks, gen_neurons))
            if len(gen_ticks) != len(gen_neurons) or len(pairs) > 10_000_000 or \
                    any(not (start <= t < start + steps and 0 <= i < count) for t, i in pairs) or \
                    any(a >= b for a, b in zip(pairs, pairs[1:])) or "spike" not in events:
                raise UnsupportedModel("invalid SpikeGeneratorGroup schedule")
        blob.u64s(gen_ticks)
        blob.u64s(gen_neurons)
        # inputs of every population program (executor.rs:1778-1821)
        tables: list = []
        inputs = {"dt": (IN_CONSTANT, dt, "f64"), "t": (IN_TIME, "f64"),
                  "N": (IN_CONSTANT, float(count), "index"), "i": (IN_INDEX, D_NEURON, "index")}
        state_index = {s["name"]: k for k, s in enumerate(pdef["states"])}
        for name, k in state_index.items():
            inputs[name] = (IN_STATE, k, D_NEURON, pdef["states"][k]["dtype"])
        if refr is not None:
            inputs["lastspike"] = (IN_LASTSPIKE, "f64")
            inputs["not_refractory"] = (IN_AVAILABLE, D_NEURON, "bool")
        _parameters(inputs, pdef["parameters"], pin["parameters"], D_NEURON, f"p{index}", tables, {})
        writable = {name: (W_NEURON, k) for name, k in state_index.items()}
        if refr is not None:
            writable["not_refractory"] = (W_AVAILABLE, 0)
        # monitor (executor.rs:1935-1980)
        monitor = pdef["monitor"]
        param_symbols = {p["name"]: p for p in pdef["parameters"]}

        def monitor_value(name):
            if name in state_index:
                blob.u(0); blob.u(DTYPES[pdef["states"][state_index[name]]["dtype"]]); blob.u(state_index[name])
            elif name in param_symbols:
                symbol = param_symbols[name]
                values = [decode_typed(v, symbol["dtype"]) for v in pin["parameters"][name]]
                if symbol["index_domain"] == "scalar":
                    blob.u(1); blob.u(DTYPES[symbol["dtype"]]); blob.f(values[0])
                else:
                    blob.u(2); blob.u(DTYPES[symbol["dtype"]]); blob.f64s(values)
            else:
                raise UnsupportedModel(f"monitor variable {name} is not a state or parameter")

        blob.u(len(monitor["variables"]))
        for name in monitor["variables"]:
            monitor_value(name)
        blob.u64s(monitor["record"])
        blob.u(1 if pdef["state_monitors"] else 0)
        # event monitors (executor.rs:3053-3080)
        event_monitors = pdef.get("event_monitors", [])
        blob.u(len(event_monitors))
        for emon in event_monitors:
            if emon["event"] not in events:
                raise UnsupportedModel(f"event monitor of an unknown event {emon['event']!r}")
            blob.u(events.index(emon["event"])); blob.u(len(emon["variables"]))
            for name in emon["variables"]:
                monitor_value(name)
        # programs, grouped by kind in code-object order
        programs = {kind: [] for kind in POP_KINDS}
        code_table = []
        for code in pdef["code_objects"]:
            kind = code["kind"]
            if kind == "poisson_input":
                # a PoissonInput runs as run_program_neurons over every neuron at its schedule
                # node (executor.rs:4121-4137), as run_regularly code does
                kind = "run_regularly"
            if kind not in POP_KINDS:
                raise UnsupportedModel(f"population code object kind {kind!r}")
            if kind in ("state_update", "subexpression_update") and programs[kind]:
                raise UnsupportedModel(f"duplicate {kind}")
            position = len(programs[kind])
            programs[kind].append(Program(code, inputs, writable, functions))
            event = code.get("event_name")
            code_table.append((POP_KINDS[kind], position, events.index(event) if event in events else -1,
                               1 if event == "spike" else 0))
        blob.u(len(tables))
        param_keys = {}
        for position, (key, (_, values)) in enumerate(tables):
            param_keys[key] = position
            blob.f64s(values)
        for kind in POP_KINDS:
            blob.u(len(programs[kind]))
            for program in programs[kind]:
                program.emit(blob, param_keys)
        blob.u(len(code_table))
        for kind, position, event, is_spike in code_table:
            blob.u(kind); blob.u(position); blob.i(event); blob.u(is_spike)

    # ---- synapses -----------------------------------------------------------------------
    blob.u(len(d["synapses"]))
    for index, (sdef, sin) in enumerate(zip(d["synapses"], inst["synapses"])):
        if sdef.get("linked_variables") or sdef.get("state_monitors"):
            raise UnsupportedModel("synapse linked variables / monitors")
        if sdef.get("source_synapse") is not None or sdef.get("target_synapse") is not None:
            raise UnsupportedModel("synapse-to-synapse projections are not supported")
        pops = d["populations"]
        spop, tpop = sdef["source_population"], sdef["target_population"]
        blob.u(spop); blob.u(tpop)
        blob.u(sdef["source_start"]); blob.u(sdef["target_start"])
        blob.u(sdef["source_count"]); blob.u(sdef["target_count"])
        topo = sin["topology"]
        generated = {}
        param_values = sin["parameters"]
        if topo["kind"] == "binary_csr":
            # the file's edges enter as an explicit topology (executor.rs:35-57)
            source, target, columns = _read_binary_csr(topo, sdef["source_count"], sdef["target_count"])
            if sdef["states"] or any(p["kind"] != "pre" or len(p["delay"]) != 1 for p in sin["pathways"]):
                raise UnsupportedModel("invalid binary CSR mapping/pathway")
            blob.u(0)
            blob.u64s(source)
            blob.u64s(target)
            edge_count = len(source)
            param_values = dict(param_values)
            for name, column in topo["initializers"].items():
                param_values[name] = [struct.pack(">d", v).hex() for v in columns[int(column)]]
        elif topo["kind"] == "explicit":
            blob.u(0)
            blob.u64s([int(v) for v in sin["source"]])
            blob.u64s([int(v) for v in sin["target"]])
            edge_count = len(sin["source"])
        elif topo["kind"] in ("fixed_total", "fixed_indegree"):
            blob.u(1 if topo["kind"] == "fixed_total" else 2)
            edge_count = topo["edge_count"]
            blob.u(edge_count); blob.u(topo.get("indegree", 0)); blob.u(int(topo["seed"]))
            names = sorted(topo["initializers"])
            blob.u(len(names))
            for k, name in enumerate(names):
                _initializer(blob, topo["initializers"][name])
                generated[name] = k
        else:
            raise UnsupportedModel(f"topology kind {topo['kind']!r}")
        blob.u(len(sdef["states"]))
        for symbol in sdef["states"]:
            values = sin["initial_state"][symbol["name"]]
            if len(values) != edge_count:
                raise UnsupportedModel("synapse state length must equal the edge count")
            encode_state(blob, symbol["dtype"], values)
        sdt = decode_f64(pops[spop]["dt"])
        spdef, tpdef = pops[spop], pops[tpop]
        inputs = {"dt": (IN_CONSTANT, sdt, "f64"), "t": (IN_TIME, "f64"),
                  "N": (IN_CONSTANT, float(edge_count), "index"),
                  "N_pre": (IN_CONSTANT, float(sdef["source_count"]), "index"),
                  "N_post": (IN_CONSTANT, float(sdef["target_count"]), "index"),
                  "i": (IN_INDEX, D_PRE, "index"), "j": (IN_INDEX, D_POST, "index")}
        syn_index = {s["name"]: k for k, s in enumerate(sdef["states"])}
        for name, k in syn_index.items():
            inputs[name] = (IN_SYN, k, sdef["states"][k]["dtype"])
        sidx = {s["name"]: k for k, s in enumerate(spdef["states"])}
        tidx = {s["name"]: k for k, s in enumerate(tpdef["states"])}
        writable = {}
        for alias, state in sdef["pre_state_aliases"].items():
            inputs[alias] = (IN_PRE, sidx[state], spdef["states"][sidx[state]]["dtype"])
            writable[alias] = (W_PRE, sidx[state])
        for alias, state in sdef["post_state_aliases"].items():
            inputs[alias] = (IN_POST, tidx[state], tpdef["states"][tidx[state]]["dtype"])
            writable[alias] = (W_NEURON, tidx[state])
        for name, k in syn_index.items():
            writable[name] = (W_SYN, k)
        if tpdef.get("refractory") is not None:
            inputs["not_refractory_post"] = (IN_AVAILABLE, D_POST, "bool")
        tables = []
        _parameters(inputs, sdef["parameters"], param_values, D_EDGE, f"s{index}", tables, generated)
        post_writable = {name: (W_SYN, k) for name, k in syn_index.items()}
        for alias, state in sdef["post_state_aliases"].items():
            post_writable[alias] = (W_NEURON, tidx[state])
        blob.u(len(tables))
        param_keys = {}
        for position, (key, (kind, values)) in enumerate(tables):
            param_keys[key] = position
            if kind == "generated":
                blob.u(1); blob.u(values)
            else:
                blob.u(0); blob.f64s(values)
        # pathways (executor.rs:3755-3815)
        code_by_pathway = {}
        for code in sdef["code_objects"]:
            if code["kind"] not in ("synapses", "synapses_post", "synapse_state_update", "summed_variable"):
                raise UnsupportedModel(f"synapse code object kind {code['kind']!r}")
            if code["kind"] in ("synapses", "synapses_post"):
                code_by_pathway[code["pathway_name"]] = code
        blob.u(len(sin["pathways"]))
        for pathway in sin["pathways"]:
            is_pre = pathway["kind"] == "pre"
            code = code_by_pathway[pathway["name"]]
            endpoint = pops[spop if is_pre else tpop]
            pinputs = dict(inputs)
            pinputs["dt"] = (IN_CONSTANT, decode_f64(endpoint["dt"]), "f64")
            program = Program(code, pinputs, writable if is_pre else post_writable, functions)
            blob.u(1 if is_pre else 0)
            if pathway["event"] not in endpoint["events"]:
                raise UnsupportedModel("pathway event missing from endpoint")
            blob.u(endpoint["events"].index(pathway["event"]))
            if topo["kind"] != "explicit" and pathway.get("delay_initializer"):
                blob.u(1)
                _initializer(blob, pathway["delay_initializer"], decode_f64(endpoint["dt"]))
                blob.f(decode_f64(endpoint["dt"]))
            else:
                blob.u(0)
                blob.u64s([int(v) for v in pathway["delay_ticks"]])
            pending = pathway.get("pending", [])
            # model.rs:4322-4338: delivery ticks ascend and fall inside the endpoint's run;
            # items are endpoints for a uniform delay, edges otherwise
            delays = [int(v) for v in pathway["delay_ticks"]]
            uniform = bool(delays) and all(v == delays[0] for v in delays)
            first = run["clocks"][endpoint["clock"]]["start_tick"]
            items = (sdef["source_count"] if is_pre else sdef["target_count"]) if uniform else edge_count
            ticks = [int(e["delivery_tick"]) for e in pending]
            if (len(pending) > 10_000_000 or any(a > b for a, b in zip(ticks, ticks[1:]))
                    or any(not first <= t < first + endpoint["steps"] for t in ticks)
                    or any(not 0 <= int(e["item"]) < items for e in pending)):
                raise UnsupportedModel("invalid pending synaptic pathway event")
            blob.u(len(pending))
            for event in pending:
                blob.u(event["delivery_tick"]); blob.u(event["item"])
            program.emit(blob, param_keys)
        # every code object: 0 a pathway (its index); 1 the clock-driven state update, which writes
        # only the clock-driven synapse states (executor.rs:3607-3623, 2513-2546); 2 a summed
        # variable: the target population state it fills, the register of `_synaptic_var`, its
        # endpoint range, with dt of the target population (executor.rs:3655-3730, 2548-2597)
        blob.u(len(sdef["code_objects"]))
        names = [p["name"] for p in sin["pathways"]]
        clock_driven = list(sdef.get("clock_driven_states", []))
        if len(set(clock_driven)) != len(clock_driven) or not set(clock_driven) <= set(syn_index):
            raise UnsupportedModel("invalid clock-driven synaptic state list")
        if sum(c["kind"] == "synapse_state_update" for c in sdef["code_objects"]) != (1 if clock_driven else 0):
            raise UnsupportedModel("expected one synapse state update for the clock-driven states")
        for code in sdef["code_objects"]:
            if code["kind"] in ("synapses", "synapses_post"):
                blob.u(0)
                blob.u(names.index(code["pathway_name"]))
            elif code["kind"] == "synapse_state_update":
                blob.u(1)
                Program(code, dict(inputs), {name: (W_SYN, syn_index[name]) for name in clock_driven},
                        functions).emit(blob, param_keys)
            else:
                if code.get("when") not in ("groups", "after_groups") or code.get("pathway_name") is not None:
                    raise UnsupportedModel("pathway metadata on summed code object")
                to_pre = code.get("summed_target") == "pre"
                if code.get("summed_target") not in ("pre", "post"):
                    raise UnsupportedModel("invalid summed variable endpoint")
                endpoint = pops[spop if to_pre else tpop]
                names_ = [st["name"] for st in endpoint["states"]]
                if code.get("summed_state") not in names_:
                    raise UnsupportedModel("summed variable target must be mutable population state")
                state_index = names_.index(code["summed_state"])
                if endpoint["states"][state_index]["dtype"] not in ("f32", "f64"):
                    raise UnsupportedModel("summed variables require floating-point state")
                sinputs = dict(inputs)
                sinputs["dt"] = (IN_CONSTANT, decode_f64(endpoint["dt"]), "f64")
                program = Program(code, sinputs, {}, functions)
                if "_synaptic_var" not in program.symbols:
                    raise UnsupportedModel("missing summed expression result")
                blob.u(2)
                blob.u(1 if to_pre else 0); blob.u(state_index); blob.u(program.symbols["_synaptic_var"])
                blob.u(sdef["source_start"] if to_pre else sdef["target_start"])
                blob.u(sdef["source_count"] if to_pre else sdef["target_count"])
                program.emit(blob, param_keys)

    # ---- schedule -------------------------------------------------------------------------
    nodes = d["schedule"]["nodes"]
    if not nodes:
        raise UnsupportedModel("an empty schedule uses the legacy phase loop")
    operations = {"code_object": 0, "state_monitor": 1, "spike_monitor": 2, "event_source": 3, "event_monitor": 4}
    blob.u(len(nodes))
    for node in nodes:
        if node["operation"] not in operations:
            raise UnsupportedModel(f"schedule operation {node['operation']!r}")
        blob.u(operations[node["operation"]])
        blob.u(0 if node["owner_kind"] == "population" else 1)
        blob.u(node["owner_index"]); blob.u(node["item_index"]); blob.u(node["clock"])
    return blob.bytes()
