"""Lowering of an AtlasIR v1 document to the HIP engine: plan, buffers, generated module.

The reference GPU path derives per-stage kernels from AtlasIR in Python
(``metal.py:396-572`` population kernels, ``metal_dag.py:55-409`` delivery DAG)
and runs them through CuPy (``cuda.py:80-392``).  Here the same document lowers
to one hiprtc module per model:

* per population, a fused ``update`` device function (fixed-refractory recompute,
  state-update statements, threshold) and a ``reset`` function, generated from
  the statement trees;
* per pathway, an ``apply`` function running the on_pre program for one target
  over its events in canonical order;
* one or two tick kernels that instantiate the hand-written templates of
  ``csrc/device/atlas_tick.h``.

Numerics follow the reference CPU engine, not the reference GPU kernels: every
expression node is an f64 operation (contraction off), f32 storage rounds once
per committed statement, threshold comparisons are f64, and every arithmetic
result is checked for finiteness (executor.rs:5725-5760).  Scalar statements
(loop invariants) are evaluated once on the host with the host libm, as the
reference does in ``Program::prepare`` (executor.rs:5488-5515), and enter the
module as exact hexadecimal literals.

The supported subset is checked before anything runs; outside it the lowering
raises ``UnsupportedModel`` (AtlasIR.md section 1: a backend must reject an
unsupported valid model before creating results).
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass, field

import numpy as np

from . import native, protocol

XCDS = 8              # MI355X accelerator complex dies; workgroup i runs on XCD i mod 8
PERSISTENT_TICKS = 10_000   # ticks per cooperative launch of a persistent plan
PERSISTENT_SPLIT = True     # delay >= 1: exchange and update waves side by side (persistent_run_split)
SPLIT_XWAVES = 0            # exchange waves of the split loop (0: half the workgroup's waves)
PERSISTENT_EDGES = True     # ordered groups in the split loop through edge-keyed LDS lists (Group::EDGE)
EDGE_KEY_BITS = 30          # edge id bits of an edge-keyed event (atlas_tick.h ATLAS_EDGE_BITS)
LDS_BYTES = 160 * 1024      # LDS per CU (one workgroup of the split loop per CU)
ATLAS_XLIST = 512           # fired sources one exchange wave of the split loop keeps (atlas_tick.h)
EDGE_XLIST = 256            # the same with edge buckets (config 3 lists about 111 per wave and tick)
RESIDENT_BLOCKS = 512       # 512-wide workgroups resident at once: two per CU on 256 CUs
CUS = 256             # compute units
PATH_MAX_SOURCE_BLOCKS = 8192


@dataclass(frozen=True)
class Shape:
    """Launch shape of the tick kernels.

    block: neurons per workgroup block; wg: work-items per workgroup;
    spt: fired sources gathered per work-item per gather pass;
    cap_bits: log2 of the events staged in LDS per ordered-delivery flush.
    """
    block: int
    wg: int
    spt: int
    cap_bits: int


# Measured on the 1M-neuron configuration (us per tick, identical results):
# 1024/256 28.2, 2048/512 22.1, 4096/1024 22.5, 4096/512 27.2.
SHAPES = {2048: Shape(2048, 512, 2, 11), 1024: Shape(1024, 256, 4, 10), 512: Shape(512, 256, 4, 10),
          256: Shape(256, 256, 4, 10)}


# A persistent launch needs at least this many blocks: config 2's 16 blocks of 256 HH neurons
# measured 10.75 us per tick persistent against 13.22 with one launch per tick.
PERSISTENT_MIN_BLOCKS = 16

# One population of at least this many neurons takes 4096-neuron blocks of 1024 work-items,
# one workgroup per CU: for config 3's network (1M neurons, 245 blocks) a persistent tick then
# reads one slot per fired source per CU instead of two and exchanges half as many records
# (7.95 against 8.93 us per tick measured at in-degree 250, identical results).
LARGE_BLOCK_NEURONS = 64 * 4096


def choose_shape(total_neurons: int, populations: int = 1) -> Shape:
    """The largest block that still gives every compute unit a workgroup (at least
    CUS blocks); small networks use 256-neuron blocks, one neuron per work-item; one large
    population takes 4096-neuron blocks."""
    if populations == 1 and total_neurons >= LARGE_BLOCK_NEURONS:
        return Shape(4096, 1024, 2, 11)
    for block in (2048, 1024, 512):
        if -(-total_neurons // block) >= CUS:
            return SHAPES[block]
    return SHAPES[256]


class UnsupportedModel(ValueError):
    """Valid AtlasIR outside the HIP engine's supported subset."""


def require(condition, message: str) -> None:
    if not condition:
        raise UnsupportedModel(message)


def decode_f64(bits: str) -> float:
    return struct.unpack(">d", bytes.fromhex(bits))[0]


def decode_f32(bits: str) -> float:
    return struct.unpack(">f", bytes.fromhex(bits))[0]


def decode_array(values, dtype: str) -> np.ndarray:
    """Decode an AtlasIR hex array into storage-typed numpy values.  In-memory documents
    may carry numpy arrays in place of hex lists (packed large arrays)."""
    if isinstance(values, np.ndarray):
        return values.astype(NUMPY[dtype], copy=False) if dtype in NUMPY else values
    joined = "".join(values)
    raw = bytes.fromhex(joined)
    if dtype == "f64":
        return np.frombuffer(raw, ">f8").astype(np.float64)
    if dtype == "f32":
        return np.frombuffer(raw, ">f4").astype(np.float32)
    if dtype == "bool":
        return np.frombuffer(raw, np.uint8).astype(np.uint8)
    if dtype == "i32":
        return np.frombuffer(raw, ">i4").astype(np.int32)
    if dtype == "i64":
        return np.frombuffer(raw, ">i8").astype(np.int64)
    raise UnsupportedModel(f"unsupported array dtype {dtype}")


NUMPY = {"f32": np.float32, "f64": np.float64, "bool": np.uint8, "i32": np.int32, "i64": np.int64}
CTYPE = {"f32": "float", "f64": "double", "bool": "byte_t", "i32": "int", "i64": "i64"}


def hexlit(value: float) -> str:
    """Exact C++ literal of a finite f64 value."""
    if value == 0.0:
        return "-0.0" if math.copysign(1.0, value) < 0 else "0.0"
    require(math.isfinite(value), "non-finite constant")
    return float(value).hex()


def commit_expr(dtype: str, value: str) -> str:
    """Storage conversion of a register value (StateArray::set_register)."""
    if dtype == "f32":
        return f"(float)({value})"
    if dtype == "f64":
        return value
    if dtype == "bool":
        return f"(byte_t)(({value}) != 0.0)"
    if dtype == "i32":
        return f"(int)(i64)({value})"
    if dtype == "i64":
        return f"(i64)({value})"
    raise UnsupportedModel(f"unsupported storage dtype {dtype}")


# ----------------------------------------------------------------- host scalars
_MATH = {"exp": math.exp, "log": math.log, "log10": math.log10, "sqrt": math.sqrt, "sin": math.sin,
         "cos": math.cos, "tan": math.tan, "sinh": math.sinh, "cosh": math.cosh, "tanh": math.tanh,
         "arcsin": math.asin, "arccos": math.acos, "arctan": math.atan, "floor": math.floor,
         "ceil": math.ceil, "expm1": math.expm1, "log1p": math.log1p, "abs": abs}


def eval_scalar(expr: dict, env: dict) -> float:
    """Host f64 evaluation of a scalar statement expression (Program::prepare)."""
    op = expr["op"]
    if op == "literal":
        return decode_f64(expr["bits"])
    if op == "boolean":
        return 1.0 if expr["value"] else 0.0
    if op == "integer":
        require(expr["dtype"] in ("i32", "i64"), "unsigned integer literal in a scalar statement")
        return float(int(expr["value"]))
    if op == "load":
        require(expr["name"] in env, f"scalar statement reads {expr['name']!r}, which is not a per-run constant")
        return env[expr["name"]]
    if op in ("f32_to_f64", "bool_to_f64", "index_to_f64", "tick_to_f64"):
        return eval_scalar(expr["arg"], env)
    if op == "f64_to_f32":
        value = struct.unpack("<f", struct.pack("<f", eval_scalar(expr["arg"], env)))[0]
        require(math.isfinite(value), "non-finite scalar value")
        return value
    if op == "cast":
        value = eval_scalar(expr["arg"], env)
        require(expr["dtype"] in ("f64", "i32", "i64"), "unsupported scalar cast")
        return value if expr["dtype"] == "f64" else float(math.trunc(value))
    if op == "neg":
        return -eval_scalar(expr["arg"], env)
    if op == "not":
        return 1.0 if eval_scalar(expr["arg"], env) == 0.0 else 0.0
    if op in _MATH:
        result = float(_MATH[op](eval_scalar(expr["arg"], env)))
    elif op == "exprel":
        a = eval_scalar(expr["arg"], env)
        result = 1.0 if abs(a) < 1e-16 else (math.inf if a > 717.0 else math.expm1(a) / a)
    elif op == "clip":
        result = min(max(eval_scalar(expr["value"], env), eval_scalar(expr["min"], env)), eval_scalar(expr["max"], env))
    elif op in ("add", "sub", "mul", "div", "pow", "mod", "floordiv", "eq", "ne", "gt", "ge", "lt", "le", "and", "or"):
        a = eval_scalar(expr["left"], env)
        b = eval_scalar(expr["right"], env)
        result = {"add": lambda: a + b, "sub": lambda: a - b, "mul": lambda: a * b,
                  "div": lambda: a / b if b != 0.0 else math.copysign(math.inf, a) if a != 0 else math.nan,
                  "pow": lambda: math.pow(a, b), "mod": lambda: a - b * math.floor(a / b),
                  "floordiv": lambda: float(math.floor(a / b)),
                  "eq": lambda: float(a == b), "ne": lambda: float(a != b), "gt": lambda: float(a > b),
                  "ge": lambda: float(a >= b), "lt": lambda: float(a < b), "le": lambda: float(a <= b),
                  "and": lambda: float(a != 0 and b != 0), "or": lambda: float(a != 0 or b != 0)}[op]()
    else:
        raise UnsupportedModel(f"scalar op {op!r} is not supported")
    require(math.isfinite(result), "non-finite numeric value in a scalar statement")
    return result


# ----------------------------------------------------------------- device code
FLOAT_BINARY = {"add": "+", "sub": "-", "mul": "*", "div": "/"}
DEVICE_MATH = {"exp": "atlas_exp", "expm1": "atlas_expm1", "exprel": "atlas_exprel", "log": "atlas_log"}
COMPARE = {"eq": "==", "ne": "!=", "gt": ">", "ge": ">=", "lt": "<", "le": "<="}


class DeviceProgram:
    """Straight-line f64 code for one statement list (Program::compile/evaluate).

    ``inputs`` maps a symbol to (C expression yielding its register value, dtype);
    inputs are materialised at first use, which equals the reference's snapshot
    binding because nothing is committed before the program ends.
    """

    def __init__(self, inputs: dict, lines: list, prefix: str, indent: str = "        ", rng: tuple | None = None):
        # rng = (seed, C expression of the counter index): rand() draws counter_uniform(seed,
        # stream, tick, index) (executor.rs:190-222); None where random draws are unsupported
        self.rng = rng
        self.inputs = inputs
        self.symbols: dict[str, tuple[str, str]] = {}
        self.lines = lines
        self.prefix = prefix
        self.indent = indent
        self.count = 0
        # emitted finiteness checks not yet subsumed: var -> (line index, guard)
        self.pending: dict[str, tuple[int, str | None]] = {}
        self.edges: dict[str, tuple] = {}     # var -> operands whose non-finiteness it propagates
        self.input_var: dict[str, str] = {}   # input symbol -> the var of its value
        self.rounded32: set = set()           # vars holding an f32-rounded value

    def fresh(self) -> str:
        self.count += 1
        return f"{self.prefix}{self.count}"

    def emit(self, text: str) -> None:
        self.lines.append(self.indent + text)

    def resolve(self, name: str) -> tuple[str, str]:
        if name in self.symbols:
            return self.symbols[name]
        require(name in self.inputs, f"missing program input {name!r}")
        cexpr, dtype = self.inputs[name]
        var = self.fresh()
        self.emit(f"const double {var} = {cexpr};")
        self.symbols[name] = (var, dtype)
        self.input_var.setdefault(name, var)
        return self.symbols[name]

    def scalar_statements(self, env: dict) -> None:
        """Emit the scalar statements a host environment left for the device (random draws), with
        the counter RNG's draw index 0 of a scalar statement (executor.rs:5488-5503)."""
        statements = env.get("\0device")
        if not statements:
            return
        require(self.rng is not None, "random draws in scalar statements are supported in neuron code only")
        saved = self.rng
        self.rng = (saved[0], "0")
        self.statements(statements)
        self.rng = saved

    def check(self, var: str, guard: str | None) -> None:
        self.pending[var] = (len(self.lines), guard)
        if guard is None:
            self.emit(f"atlas::finite({var}, fault);")
        else:
            self.emit(f"if ({guard} != 0.0) atlas::finite({var}, fault);")

    def value(self, expr: str, dtype: str, guard: str | None, checked: bool,
              propagated: tuple = ()) -> tuple[str, str]:
        """Emit `var = expr`, with its finiteness check when `checked`.  `propagated` names the
        operands whose non-finite values always make expr non-finite (+, -, *, a dividend,
        f32 rounding, negation, abs, sqrt, floor, ceil): their own checks under the same guard
        are then implied by this one and dropped, which raises the same fault bit on exactly
        the same inputs."""
        var = self.fresh()
        self.emit(f"const double {var} = {expr};")
        self.edges[var] = tuple(propagated)
        if checked:
            self.check(var, guard)
            for operand in propagated:
                line = self.pending.get(operand)
                if line is not None and line[1] == guard:
                    self.lines[line[0]] = f"{self.indent}// finiteness of {operand} checked through {var}"
                    del self.pending[operand]
        return var, dtype

    def expression(self, expr: dict, guard: str | None) -> tuple[str, str]:
        op = expr["op"]
        if op == "literal":
            return hexlit(decode_f64(expr["bits"])), "f64"
        if op == "boolean":
            return ("1.0" if expr["value"] else "0.0"), "bool"
        if op == "integer":
            require(expr["dtype"] in ("i32", "i64"), "unsigned integers are not supported")
            value = int(expr["value"])
            require(abs(value) <= 2**53, "integer literal beyond the exact f64 range")
            return hexlit(float(value)), expr["dtype"]
        if op == "load":
            return self.resolve(expr["name"])
        if op == "rand":
            require(self.rng is not None, "random draws are supported in neuron update, threshold and reset code only")
            seed, index = self.rng
            return self.value(f"atlas::counter_uniform({int(seed) & (2**64 - 1)}ull, {int(expr['stream'])}ull, "
                              f"(u64)tick, (u64)({index}))", "f64", guard, False)
        if op == "randn":
            # counter_normal (executor.rs:200-222): the polar method on the stream's draws
            require(self.rng is not None, "random draws are supported in neuron code only")
            seed, index = self.rng
            return self.value(f"atlas::counter_normal({int(seed) & (2**64 - 1)}ull, {int(expr['stream'])}ull, "
                              f"(u64)tick, (u64)({index}), fault)", "f64", guard, False)
        if op == "poisson":
            # counter_poisson (executor.rs:290-323, 6086-6101): NaN for an invalid rate, which the
            # finiteness check reports as the reference's error
            require(self.rng is not None, "random draws are supported in neuron code only")
            require(0 <= int(expr["stream"]) < 1_000_000, "invalid poisson expression")
            lam, _ = self.expression(expr["lambda"], guard)
            seed, index = self.rng
            call = (f"atlas::counter_poisson({int(seed) & (2**64 - 1)}ull, {int(expr['stream'])}ull, (u64)tick, "
                    f"(u64)({index}), {lam}, fault)")
            if guard is not None:
                call = f"(({guard}) != 0.0 ? {call} : 0.0)"
            return self.value(call, "f64", guard, True)
        if op == "binomial":
            # counter_binomial (executor.rs:224-268, 6063-6084); only lanes whose statement runs draw
            require(self.rng is not None, "random draws are supported in neuron code only")
            n, stream = int(expr["n"]), int(expr["stream"])
            require(1 <= n <= 2**31 - 1 and 0 <= stream < 1_000_000, "invalid binomial expression")
            p, _ = self.expression(expr["p"], guard)
            seed, index = self.rng
            call = (f"atlas::counter_binomial({int(seed) & (2**64 - 1)}ull, {stream}ull, (u64)tick, (u64)({index}), "
                    f"{n}ull, {p}, {'true' if expr.get('approximate') else 'false'}, fault)")
            if guard is not None:
                call = f"(({guard}) != 0.0 ? {call} : 0.0)"
            return self.value(call, "f64", guard, False)
        if op in ("f32_to_f64", "bool_to_f64", "index_to_f64", "tick_to_f64"):
            value, _ = self.expression(expr["arg"], guard)
            return value, "f64"
        if op == "f64_to_f32":
            arg, _ = self.expression(expr["arg"], guard)
            out = self.value(f"(double)(float)({arg})", "f32", guard, True, (arg,))
            self.rounded32.add(out[0])
            return out
        if op == "cast":
            arg, source = self.expression(expr["arg"], guard)
            target = expr["dtype"]
            if target == "f64":
                require(source in ("f64", "f32", "bool", "i32", "i64"), f"cast from {source}")
                return arg, "f64"
            require(target in ("i32", "i64"), f"cast to {target} is not supported")
            if source == "bool":
                return self.value(f"(({arg}) != 0.0 ? 1.0 : 0.0)", target, guard, False)
            if source in ("f64", "f32"):
                return self.value(f"atlas::saturate_{target}({arg})", target, guard, False)
            if source in ("i32", "i64"):
                return self.value(f"atlas::wrap_{target}({arg})", target, guard, False)
            raise UnsupportedModel(f"cast from {source}")
        if op == "neg":
            arg, dtype = self.expression(expr["arg"], guard)
            require(dtype == "f64", "integer negation is not supported")
            return self.value(f"-({arg})", "f64", guard, True, (arg,))
        if op == "abs":
            arg, dtype = self.expression(expr["arg"], guard)
            require(dtype == "f64", "integer abs is not supported")
            return self.value(f"fabs({arg})", "f64", guard, True, (arg,))
        if op == "not":
            arg, _ = self.expression(expr["arg"], guard)
            return self.value(f"(({arg}) == 0.0 ? 1.0 : 0.0)", "bool", guard, False)
        if op in DEVICE_MATH:
            # the shared correctly rounded implementation (atlas_math.h), also used by the
            # oracle's shared-math mode; the reference calls the host libm here
            arg, _ = self.expression(expr["arg"], guard)
            return self.value(f"{DEVICE_MATH[op]}({arg})", "f64", guard, True)
        if op in ("sqrt", "floor", "ceil"):
            arg, _ = self.expression(expr["arg"], guard)
            return self.value(f"{op}({arg})", "f64", guard, True, (arg,))
        if op in FLOAT_BINARY or op in ("mod", "floordiv"):
            left_dtype = self._dtype(expr["left"])
            require(left_dtype not in ("i32", "i64"), "integer arithmetic is not supported")
            a, _ = self.expression(expr["left"], guard)
            b, _ = self.expression(expr["right"], guard)
            propagated = ()
            if op in FLOAT_BINARY:
                text = f"{a} {FLOAT_BINARY[op]} {b}"
                # a finite value divided by an infinite one is zero: only the dividend propagates
                propagated = (a,) if op == "div" else (a, b)
            elif op == "mod":
                text = f"{a} - {b} * floor({a} / {b})"
            else:
                text = f"floor({a} / {b})"
            return self.value(text, "f64", guard, True, propagated)
        if op in COMPARE:
            a, _ = self.expression(expr["left"], guard)
            b, _ = self.expression(expr["right"], guard)
            return self.value(f"(({a}) {COMPARE[op]} ({b}) ? 1.0 : 0.0)", "bool", guard, False)
        if op in ("and", "or"):
            a, _ = self.expression(expr["left"], guard)
            b, _ = self.expression(expr["right"], guard)
            joiner = "&&" if op == "and" else "||"
            return self.value(f"((({a}) != 0.0 {joiner} ({b}) != 0.0) ? 1.0 : 0.0)", "bool", guard, False)
        if op == "clip":
            v, _ = self.expression(expr["value"], guard)
            lo, _ = self.expression(expr["min"], guard)
            hi, _ = self.expression(expr["max"], guard)
            return self.value(f"fmin(fmax({v}, {lo}), {hi})", "f64", guard, True)
        raise UnsupportedModel(f"expression op {op!r} is not supported on the HIP engine")

    def _dtype(self, expr: dict) -> str:
        op = expr["op"]
        if op == "load":
            if expr["name"] in self.symbols:
                return self.symbols[expr["name"]][1]
            return self.inputs.get(expr["name"], ("", "f64"))[1]
        if op in ("integer", "cast"):
            return expr["dtype"]
        if op in ("add", "sub", "mul"):
            left = self._dtype(expr["left"])
            return left if left in ("i32", "i64") and left == self._dtype(expr["right"]) else "f64"
        return "f64"

    def propagates(self, source: str, target: str) -> bool:
        """Whether a non-finite `source` always makes `target` non-finite (a chain of
        propagating operations)."""
        stack, seen = [target], set()
        while stack:
            var = stack.pop()
            if var == source:
                return True
            if var not in seen:
                seen.add(var)
                stack.extend(self.edges.get(var, ()))
        return False

    def statements(self, statements: list) -> None:
        for statement in statements:
            condition = statement.get("condition")
            guard = self.resolve(condition)[0] if condition is not None else None
            old = None
            target = statement["target"]
            if guard is not None:
                if target in self.symbols:
                    old = self.symbols[target][0]
                elif target in self.inputs:
                    old = self.resolve(target)[0]
            value, _ = self.expression(statement["value"], guard)
            if old is not None:
                var = self.fresh()
                self.emit(f"const double {var} = ({guard} != 0.0) ? {value} : {old};")
                value = var
            self.symbols[target] = (value, statement["dtype"])


# ---------------------------------------------------------------------- plans
@dataclass
class Buffer:
    name: str
    nbytes: int
    init: np.ndarray | None = None


@dataclass
class PopulationPlan:
    index: int
    name: str
    count: int
    blocks: int
    first_block: int
    dt: float
    steps: int
    start_tick: int
    states: list             # (name, dtype, np array)
    scalar_params: dict      # name -> (dtype, value)
    vector_params: dict      # name -> (dtype, np.ndarray f64 registers)
    refractory: tuple | None  # (period_ticks, lastspike f64[n], not_refractory u8[n], until i32[n])
    update: dict | None
    threshold: dict | None
    reset: dict | None
    events: list
    spike_monitor: bool
    monitor_vars: list
    monitor_record: list
    window_start: int
    ring: int = 1
    reset_fused: bool = False
    lds_states: dict = field(default_factory=dict)  # state -> byte offset in the LDS post area
    fused_counts: bool = False                       # counted events applied inside phase_a_run
    fused_split: bool = False                        # delay-0 plans: the previous tick's counts applied in registers
    fused_edges: bool = False                        # an ordered group's edge-keyed lists applied in registers (split loop)
    fused_writes: set = field(default_factory=set)   # states those events write
    clock: int = 0                  # index of the population's clock
    buffers: dict = field(default_factory=dict)
    scalar_values: dict = field(default_factory=dict)
    generator: tuple | None = None   # SpikeGeneratorGroup: (per-neuron offsets u32[n+1], spike ticks u32)
    event_monitors: list = field(default_factory=list)   # (name, variables, event, when) of EventMonitors
    # custom events (NeuronGroup events=..., run_on_event): (name, threshold code, reset code or None)
    custom_events: list = field(default_factory=list)
    reset_order: list = field(default_factory=list)       # event names of the reset nodes, in schedule order
    # custom event index -> ticks of its ring of fired neurons, for the pathways that event triggers
    event_rings: dict = field(default_factory=dict)
    event_capacity: int = 0                               # events a run can produce (count x steps)
    poisson_inputs: list = field(default_factory=list)    # PoissonInput code objects, in schedule order
    # run_regularly code objects in schedule order with their place in the tick: "pre" (before the
    # update), "mid" (after the update, before the threshold) or "end" (after the reset)
    regular: list = field(default_factory=list)

    def event_monitor_capacity(self, k: int) -> int:
        """Records EventMonitor k may hold: the reference's budget (executor.rs:3061-3066), at most
        10M events and 10M samples, and no more than the run can produce."""
        return min(self.event_capacity, EVENT_MONITOR_BUDGET // max(1, len(self.event_monitors[k][1])))

    @property
    def has_spike_event(self) -> bool:
        return "spike" in self.events


@dataclass
class PathwayPlan:
    index: int
    synapse: int
    name: str
    code: dict
    source: int
    target: int
    sstart: int
    scount: int
    tstart: int
    tcount: int
    topology: tuple          # ("explicit", src, tgt) | ("fixed_indegree", K, seed)
    edge_count: int
    delays: np.ndarray       # per-edge ticks or a single uniform entry
    dvals: list              # distinct delays, descending
    edge_params: dict        # name -> (dtype, f64 values per edge, or None when generated)
    scalar_params: dict      # name -> (dtype, value)
    syn_states: list         # (name, dtype, values per edge)
    post_aliases: dict
    buffers: dict = field(default_factory=dict)
    event: str = "spike"              # the source population's event that triggers the pathway
    # another on_pre pathway of the same Synapses whose rows hold the synapse states this one
    # touches (reached through the rec_row map), or None
    state_owner: "PathwayPlan | None" = None
    order: np.ndarray | None = None   # row position -> edge id (explicit layouts)
    random: bool = False              # a program of the projection draws from the counter RNG
    slot_entries: int = 0             # slot-table entries (counting groups): XCDS x groups x per_xcd
    syn_fields: dict = field(default_factory=dict)   # synapse state -> (byte offset, dtype) in its row's record
    syn_stride: int = 0                              # bytes per row record of the synapse states
    pending: tuple | None = None    # (tick offset, item, uniform): events inherited from the previous run
    pending_ticks: int = 0          # ticks of the group's pending-event table (group's first pathway)
    pending_sources: bool = False   # the table lists pending sources per tick (counting pull groups)
    row_slots: bool = False         # slot table with the first row in every slot (edge-keyed lists)
    # rows ordered by target (post_major_paths): the segment and target tables then list the
    # out-edges in source-major positions, and out_row maps a position to its row
    post_major: bool = False
    # per-edge parameters drawn by a procedural uniform initializer on a device topology, evaluated
    # from the row (= edge id) where read: name -> (seed, stream, minimum, maximum)
    edge_gen: dict = field(default_factory=dict)


@dataclass
class PostPlan:
    """An on_post pathway: spikes of the synapse's target population, after a uniform
    delay, run the program once per incoming edge of the spiking neuron.  It writes
    only synapse states (stored in the rows of the synapse's pre pathway)."""
    index: int               # delivered-counter row (after the pre pathways)
    synapse: int
    name: str
    code: dict
    pre: "PathwayPlan"       # the synapse's pre pathway (rows, synapse-state buffers)
    delay: int
    buffers: dict = field(default_factory=dict)
    pending: tuple | None = None    # (tick offset, target item, True): events inherited from the previous run
    pending_ticks: int = 0
    event: str = "spike"            # the target population's event that triggers the pathway
    dvals: list = field(default_factory=list)   # distinct delays, descending (delay is the largest)
    delays: np.ndarray | None = None            # per-edge delays when there are several


@dataclass
class SynCodePlan:
    """A synapse code object run over every edge once per tick before the tick kernel: the
    clock-driven state update (kind "update": each edge's clock-driven synapse states, rows in
    any order since an edge reads and writes only its own) or a summed variable (kind "summed":
    a population state over the endpoint range set to the sum, in edge order, of every incoming
    edge's `_synaptic_var`)."""
    kind: str
    synapse: int
    code: dict
    path: "PathwayPlan"            # the synapse's pre pathway (rows, per-edge buffers)
    to_pre: bool = False           # summed into the source population (else the target)
    state: str = ""                # summed population state
    dtype: str = "f64"             # its dtype
    population: int = -1           # its population
    start: int = 0                 # endpoint range [start, start + count) of the population
    count: int = 0
    buffers: dict = field(default_factory=dict)


@dataclass
class Plan:
    document: dict
    populations: list
    pathways: list
    synapse_count: int
    synapse_edges: list
    dt: float
    start_tick: int
    steps: int
    split: bool
    shape: Shape = SHAPES[256]
    post_paths: list = field(default_factory=list)
    buffers: list = field(default_factory=list)
    source: str = ""
    kernels: list = field(default_factory=list)
    launches: list = field(default_factory=list)
    total_blocks: int = 0
    groups: list = field(default_factory=list)
    fault_buffer: int = 0
    delivered_buffer: int = 0
    slot_fallback: set = field(default_factory=set)   # pathways whose slot table overflowed
    queues: dict = field(default_factory=dict)        # queued groups: first pathway index -> capacities
    rng_seed: int = 0                                 # the instance's counter-RNG seed
    epilogue: list = field(default_factory=list)      # launches once after the last tick of a run
    persistent: tuple | None = None                   # (kernel, grid, work-items, LDS) of atlas_run, if eligible
    barrier_buffer: int = 0                           # grid-barrier words of persistent launches
    synapse_codes: list = field(default_factory=list)  # SynCodePlans in schedule order (run before each tick)
    # several clocks: per step of the merged run, each clock's tick, or -1 where it does not advance
    clock_table: np.ndarray | None = None
    clocks: list = field(default_factory=list)       # (dt, start tick, steps) of each clock
    clock_buffer: int = -1
    edge_nodes: int = 0                              # events the split loop's edge buckets hold per workgroup and tick

    @property
    def multi_clock(self) -> bool:
        return self.clock_table is not None

    def end_tick(self, pop: "PopulationPlan", steps: int) -> int:
        """The population's tick after the first ``steps`` steps of the run."""
        if self.clock_table is None:
            return self.start_tick + steps
        return pop.start_tick + int((self.clock_table[:steps, pop.clock] >= 0).sum())

    def add(self, name: str, nbytes: int, init: np.ndarray | None = None) -> int:
        self.buffers.append(Buffer(name, int(nbytes), init))
        return len(self.buffers) - 1

    @property
    def sha256(self) -> str:
        import hashlib
        return hashlib.sha256(self.source.encode()).hexdigest()


# ------------------------------------------------------------------- lowering
POP_KINDS = {"state_update", "threshold", "reset", "poisson_input", "run_regularly"}


def _register_values(values, dtype: str) -> np.ndarray:
    arr = decode_array(values, dtype)
    return arr.astype(np.float64)


def _initializer_values(spec: dict, count: int, seed: int, delay_dt: float | None = None) -> np.ndarray:
    """Per-edge values of a procedural initializer (executor.rs:139-188): a delay initializer
    (``delay_dt`` given) clips a clipped normal to [max(minimum or 0, 0), maximum or dt * 1e6]."""
    kind = spec["kind"]
    require(kind in ("uniform", "clipped_normal"), f"initializer {kind!r} is not supported")
    stream = int(spec["stream"])
    try:
        if kind == "uniform":
            return native.prepare_initializer(0, count, seed, stream, decode_f64(spec["minimum"]),
                                              decode_f64(spec["maximum"]))
        low = decode_f64(spec["minimum"]) if spec.get("minimum") is not None else None
        high = decode_f64(spec["maximum"]) if spec.get("maximum") is not None else None
        if delay_dt is not None:
            low = max(0.0 if low is None else low, 0.0)
            high = delay_dt * 1_000_000.0 if high is None else high
        return native.prepare_initializer(1, count, seed, stream, 0.0 if low is None else low,
                                          0.0 if high is None else high, decode_f64(spec["mean"]),
                                          decode_f64(spec["std"]), low is not None, high is not None)
    except native.PrepareError as error:
        raise UnsupportedModel(str(error)) from None


def _prepare_procedural(d: dict, sdef: dict, sin: dict):
    """A fixed-in-degree or fixed-total projection with its initializers, materialised on the host
    (materialize_projection, executor.rs:19-137): source-major local (source, target) int64 arrays,
    the generated per-edge parameters, and each pathway's delay ticks (a delay initializer's
    values quantised as floor(delay / dt + 0.5), saturated to >= 0 as Rust's `as usize` does)."""
    topo = sin["topology"]
    seed = int(topo["seed"]) & (2**64 - 1)
    edges = int(topo["edge_count"])
    try:
        if topo["kind"] == "fixed_total":
            src, tgt = native.prepare_fixed_total(sdef["source_count"], sdef["target_count"], edges, seed)
        else:
            require(edges == int(topo["indegree"]) * sdef["target_count"], "fixed-indegree edge count mismatch")
            src, tgt = native.prepare_fixed_indegree(sdef["source_count"], sdef["target_count"],
                                                     int(topo["indegree"]), seed)
    except native.PrepareError as error:
        raise UnsupportedModel(str(error)) from None
    columns = {name: _initializer_values(spec, edges, seed) for name, spec in topo["initializers"].items()}
    delays = []
    for pw in sin["pathways"]:
        spec = pw.get("delay_initializer")
        if spec is None:
            delays.append(np.asarray(pw["delay_ticks"], np.int64))
            continue
        endpoint = d["populations"][sdef["source_population"] if pw["kind"] == "pre" else sdef["target_population"]]
        dt = decode_f64(endpoint["dt"])
        values = _initializer_values(spec, edges, seed, delay_dt=dt)
        with np.errstate(invalid="ignore", over="ignore"):
            ticks = np.floor(values / dt + 0.5)
        ticks = np.where(np.isnan(ticks), 0.0, np.clip(ticks, 0.0, 2.0**62))
        delays.append(ticks.astype(np.int64))
    return src.astype(np.int64), tgt.astype(np.int64), columns, delays


def lower(source, *, verify_envelope: bool = True, shape: Shape | None = None) -> Plan:
    """Validate the supported subset and build the plan (no device work).

    ``shape`` overrides the launch shape chosen from the network size."""
    doc = protocol.load(source, verify_envelope=verify_envelope)
    d, inst, run = doc["definition"], doc["instance"], doc["run"]
    if shape is None:
        shape = choose_shape(sum(int(p["count"]) for p in d["populations"]), len(d["populations"]))
    BLOCK = shape.block
    require(d["numeric_profile"] == "reference-f64", "numeric profile must be reference-f64")
    require(len(d["clocks"]) == len(run["clocks"]) >= 1, "every clock needs its run range")
    require(not d["functions"], "user Functions are not supported")
    clocks = [(decode_f64(c["dt"]), int(r["start_tick"]), int(r["steps"])) for c, r in zip(d["clocks"], run["clocks"])]
    require(all(dt_ > 0 for dt_, _, _ in clocks), "clock dt must be positive")
    multi = len(clocks) > 1
    dt, start_tick, steps = clocks[0]
    populations = []
    first_block = 0
    for p, (pdef, pin) in enumerate(zip(d["populations"], inst["populations"])):
        require(0 <= pdef["clock"] < len(clocks), "population clock out of range")
        dt, start_tick, steps = clocks[pdef["clock"]]
        require(decode_f64(pdef["dt"]) == dt and pdef["steps"] == steps, "population clock must equal its run clock")
        require(all(m["clock"] == pdef["clock"] for m in pdef.get("state_monitors", [])),
                "state monitors on another clock than their population's are not supported")
        require(not pdef.get("linked_variables"), "linked variables are not supported")
        require(not pdef.get("spatial"), "spatial neurons are not supported")
        # a PopulationRateMonitor is a layout over the spike monitor (model.rs:3379-3386); the
        # executor records nothing more for it, and its rates come from the recorded spikes
        names = [m["name"] for m in pdef.get("rate_monitors", [])]
        require(len(set(names)) == len(names) and all(m["dtype"] in ("f32", "f64") for m in pdef.get("rate_monitors", []))
                and (not names or pdef.get("spike_monitor") is not None), "invalid rate monitor layout")
        for emon in pdef.get("event_monitors", []):
            require(emon["event"] in pdef["events"] and emon["when"] in ("thresholds", "end")
                    and emon["clock"] == pdef["clock"],
                    "event monitors record a population event at the thresholds or end slot")
        require(not pdef.get("monitor_expressions") and not pdef.get("monitor_timed_arrays"),
                "monitor expressions are not supported")
        count = pdef["count"]
        require(count > 0, "empty populations are not supported")
        generator = None
        if pin.get("spike_generator") is not None:
            generator = spike_generator_schedule(pin["spike_generator"], count, start_tick, steps)
            require(not pdef["code_objects"] and not pdef["states"] and pdef.get("refractory") is None,
                    "a spike generator population has no code objects, states or refractoriness")
        states = []
        for symbol in pdef["states"]:
            require(symbol["dtype"] in ("f32", "f64", "bool"), f"state dtype {symbol['dtype']}")
            arr = decode_array(pin["initial_state"][symbol["name"]], symbol["dtype"]).astype(NUMPY[symbol["dtype"]])
            require(arr.size == count, "state length must equal the population size")
            states.append((symbol["name"], symbol["dtype"], arr))
        scalar_params, vector_params = {}, {}
        for symbol in pdef["parameters"]:
            require(symbol["dtype"] in ("f32", "f64", "bool"), f"parameter dtype {symbol['dtype']}")
            values = _register_values(pin["parameters"][symbol["name"]], symbol["dtype"])
            if symbol["index_domain"] == "scalar":
                scalar_params[symbol["name"]] = (symbol["dtype"], float(values[0]))
            else:
                vector_params[symbol["name"]] = (symbol["dtype"], values)
        refractory = None
        if pdef.get("refractory") is not None:
            require(pdef["refractory"]["mode"] == "fixed", "only fixed refractoriness is supported")
            r = pin["refractory"]
            lastspike = decode_array(r["initial_lastspike"], "f64").copy()
            refractory = (int(r["period_ticks"]), lastspike, np.asarray(r["initial_not_refractory"], np.uint8),
                          initial_until(lastspike, start_tick, dt, int(r["period_ticks"])))
        codes = {}
        custom: dict = {}
        poisson_inputs = []
        regular = []
        for code in pdef["code_objects"]:
            require(code["kind"] in POP_KINDS, f"population code object {code['kind']!r} is not supported")
            if code["kind"] == "run_regularly":
                # run_program_neurons over every neuron at the node's schedule position
                # (executor.rs:4139-4148); placed against the update, threshold and reset below
                require(code.get("adaptive") is None, "adaptive run_regularly code is not supported")
                require(set(code["effects"]["writes"]) <= {s_[0] for s_ in states},
                        "run_regularly code writes population states only")
                require(code["clock"] == pdef["clock"], "run_regularly code on its own clock is not supported")
                regular.append(code)
                continue
            if code["kind"] == "poisson_input":
                # PoissonInput (export.py:571-608): per neuron, state += binomial(N, rate dt) * weight
                require(not code["scalar"] and code.get("adaptive") is None,
                        "PoissonInput code with scalar statements is not supported")
                require(set(code["effects"]["writes"]) <= {s_[0] for s_ in states},
                        "a PoissonInput writes population states only")
                poisson_inputs.append(code)
                continue
            if code["kind"] in ("threshold", "reset") and code.get("event_name") != "spike":
                # a custom event: its condition at the thresholds slot and its run_on_event code at the
                # resets slot (executor.rs:4098-4118, 4157-4186)
                event = code.get("event_name")
                require(event in pdef["events"], "a threshold or reset of an undeclared event")
                entry = custom.setdefault(event, {})
                require(code["kind"] not in entry, f"more than one {code['kind']} of event {event!r}")
                require(code.get("adaptive") is None and not code["scalar"],
                        "custom event code with scalar statements is not supported")
                if code["kind"] == "threshold":
                    require(not _reads(code) & {"not_refractory", "lastspike"},
                            "custom event conditions reading refractoriness are not supported")
                else:
                    require(set(code["effects"]["writes"]) <= {s_[0] for s_ in states},
                            "run_on_event code writes population states only")
                entry[code["kind"]] = code
                continue
            require(code["kind"] not in codes, f"more than one {code['kind']} code object")
            require(code.get("adaptive") is None, "adaptive integrators are not supported")
            if code["kind"] in ("threshold", "reset"):
                require(code.get("event_name") == "spike", "only the spike event is supported")
            if code["kind"] != "state_update":
                require(not code["scalar"] or code["kind"] == "reset", "scalar statements in threshold")
            codes[code["kind"]] = code
            if code["kind"] == "state_update" and refractory is not None:
                require("not_refractory" not in code["effects"]["writes"],
                        "state updaters writing not_refractory are not supported")
        events = list(pdef["events"])
        require(len(set(events)) == len(events) and
                set(events) == ({"spike"} if "threshold" in codes or generator is not None else set()) | set(custom)
                and all("threshold" in entry for entry in custom.values()),
                "every event needs one threshold (and at most one reset)")
        require(not custom or generator is None, "a spike generator has no custom events")
        monitor = pdef["monitor"]
        window = monitor["window_steps"]
        window_start = start_tick + steps - window if window < steps else start_tick
        for name in monitor["variables"]:
            require(name in {s[0] for s in states} or name in scalar_params or name in vector_params,
                    f"monitor variable {name} is not a state or parameter")
        blocks = (count + BLOCK - 1) // BLOCK
        populations.append(PopulationPlan(
            index=p, name=pdef["name"], count=count, blocks=blocks, first_block=first_block, dt=dt, steps=steps,
            start_tick=start_tick, clock=pdef["clock"], states=states, scalar_params=scalar_params,
            vector_params=vector_params,
            refractory=refractory, update=codes.get("state_update"), threshold=codes.get("threshold"),
            reset=codes.get("reset"), events=events, spike_monitor=pdef.get("spike_monitor") is not None,
            monitor_vars=list(monitor["variables"]), monitor_record=[int(i) for i in monitor["record"]],
            window_start=window_start, generator=generator, poisson_inputs=poisson_inputs,
            regular=[(code, None) for code in regular],
            event_monitors=[(e["name"], list(e["variables"]), e["event"], e["when"])
                            for e in pdef.get("event_monitors", [])],
            custom_events=[(name, custom[name]["threshold"], custom[name].get("reset"))
                           for name in events if name in custom],
            event_capacity=count * steps))
        for _, variables, _, _ in populations[-1].event_monitors:
            for name in variables:
                require(name in {s_[0] for s_ in states} or name in scalar_params or name in vector_params,
                        f"event monitor variable {name} is not a state or parameter")
        first_block += blocks
    pathways = []
    synapse_edges = []
    post_paths: list[PostPlan] = []
    synapse_codes: list[SynCodePlan] = []
    for s, (sdef, sin) in enumerate(zip(d["synapses"], inst["synapses"])):
        require(not sdef.get("linked_variables") and not sdef.get("state_monitors"), "synapse monitors/links")
        require(sdef.get("source_synapse") is None and sdef.get("target_synapse") is None,
                "synapse-to-synapse projections are not supported")
        other_codes = [c for c in sdef["code_objects"] if c["kind"] not in ("synapses", "synapses_post")]
        kinds = [pw["kind"] for pw in sin["pathways"]]
        pres = [pw for pw in sin["pathways"] if pw["kind"] == "pre"]
        posts = [pw for pw in sin["pathways"] if pw["kind"] == "post"]
        # pathways ordered by kind, then name (model.rs:4299-4305)
        require(pres and kinds == ["pre"] * len(pres) + ["post"] * len(posts) and len(posts) <= 1,
                "a Synapses needs on_pre pathways and at most one on_post pathway")
        pathway = pres[0]
        post_pathway = posts[0] if posts else None
        code_of = {}
        source_events = d["populations"][sdef["source_population"]]["events"]
        for pw in sin["pathways"]:
            if pw["kind"] == "post":
                require(pw["event"] in d["populations"][sdef["target_population"]]["events"],
                        "pathway event missing from its target population")
            else:
                require(pw["event"] in source_events, "pathway event missing from its source population")
            codes = [c for c in sdef["code_objects"] if c.get("pathway_name") == pw["name"]]
            require(len(codes) == 1 and codes[0]["kind"] == ("synapses" if pw["kind"] == "pre" else "synapses_post"),
                    "each pathway needs exactly one code object")
            require(not codes[0]["scalar"], "scalar statements in a pathway are not supported")
            code_of[pw["name"]] = codes[0]
        require(len(sdef["code_objects"]) == len(kinds) + len(other_codes),
                "each pathway needs exactly one code object")
        require(len(pres) == 1 or sin["topology"]["kind"] == "explicit",
                "several on_pre pathways need an explicit topology")
        topo = sin["topology"]
        columns, generated = {}, {}
        prepared_delays = None
        if topo["kind"] == "binary_csr":
            src, tgt, columns = _binary_csr(sdef, sin)
            edge_count = src.size
            topology = ("explicit", src, tgt)
            delays = np.asarray(pathway["delay_ticks"], np.int64)
        elif topo["kind"] == "explicit":
            src = np.asarray(sin["source"], np.int64)
            tgt = np.asarray(sin["target"], np.int64)
            edge_count = src.size
            topology = ("explicit", src, tgt)
            require(not np.any((src < 0) | (src >= sdef["source_count"]) | (tgt < 0) | (tgt >= sdef["target_count"])),
                    "explicit topology index out of range")
            delays = np.asarray(pathway["delay_ticks"], np.int64)
        elif topo["kind"] in ("fixed_indegree", "fixed_total") and (
                topo["kind"] == "fixed_total" or other_codes or post_pathway is not None
                or any(spec["kind"] != "uniform" for spec in topo["initializers"].values())
                or any(pw.get("delay_initializer") is not None for pw in sin["pathways"])):
            # materialised on the host as the reference prepares procedural projections for its GPU
            # engines (gpu_initialization.prepare_model): an explicit topology from here on (the
            # edge lists of summed variables need the edges on the host too)
            src, tgt, columns, prepared_delays = _prepare_procedural(d, sdef, sin)
            edge_count = src.size
            topology = ("explicit", src, tgt)
            delays = prepared_delays[0]
        elif topo["kind"] == "fixed_indegree":
            edge_count = int(topo["edge_count"])
            require(edge_count == topo["indegree"] * sdef["target_count"], "fixed-indegree edge count mismatch")
            topology = ("fixed_indegree", int(topo["indegree"]), int(topo["seed"]))
            # uniform initializers stay procedural: the device topology's rows are the reference's
            # source-major edge order (checked when it is built), so each value is a function of
            # its row (materialize_uniform, large_topology.rs:129-142)
            for name, spec in topo["initializers"].items():
                low, high = decode_f64(spec["minimum"]), decode_f64(spec["maximum"])
                require(np.isfinite(low) and np.isfinite(high) and low <= high, "invalid uniform initializer")
                generated[name] = (int(topo["seed"]) & (2**64 - 1), int(spec["stream"]), low, high)
            delays = np.asarray(pathway["delay_ticks"], np.int64)
            require(delays.size == 1, "fixed-indegree projections need a uniform delay")
        else:
            raise UnsupportedModel(f"topology {topo['kind']!r} is not supported")
        require(delays.size in (1, edge_count), "delay array length")
        spop = populations[sdef["source_population"]]
        synapse_edges.append(edge_count)
        edge_params, scalar_params, edge_gen = {}, {}, {}
        for symbol in sdef["parameters"]:
            require(symbol["dtype"] in ("f32", "f64"), f"synapse parameter dtype {symbol['dtype']}")
            if symbol["name"] in generated:
                require(symbol["index_domain"] != "scalar", "an initializer draws a scalar parameter")
                seed_, stream_, low, high = generated[symbol["name"]]
                if low == high:   # lo + 0 * u: every edge holds lo
                    scalar_params[symbol["name"]] = (symbol["dtype"], low)
                else:
                    edge_params[symbol["name"]] = (symbol["dtype"], None)
                    edge_gen[symbol["name"]] = generated[symbol["name"]]
                continue
            values = columns[symbol["name"]] if symbol["name"] in columns else \
                _register_values(sin["parameters"][symbol["name"]], symbol["dtype"])
            if symbol["index_domain"] == "scalar":
                scalar_params[symbol["name"]] = (symbol["dtype"], float(values[0]))
            else:
                require(values.size == edge_count, "per-edge parameter length")
                bits = values.view(np.uint64)
                if values.size and np.all(bits == bits[0]):
                    # every edge holds the same value: a per-tick constant of the programs
                    scalar_params[symbol["name"]] = (symbol["dtype"], float(values[0]))
                else:
                    edge_params[symbol["name"]] = (symbol["dtype"], values)
        syn_states = []
        for symbol in sdef["states"]:
            require(symbol["dtype"] in ("f32", "f64"), f"synapse state dtype {symbol['dtype']}")
            arr = decode_array(sin["initial_state"][symbol["name"]], symbol["dtype"]).astype(NUMPY[symbol["dtype"]])
            require(arr.size == edge_count, "synapse state length")
            syn_states.append((symbol["name"], symbol["dtype"], arr))
        require(sdef["source_start"] + sdef["source_count"] <= d["populations"][sdef["source_population"]]["count"],
                "source range outside the population")
        require(sdef["target_start"] + sdef["target_count"] <= d["populations"][sdef["target_population"]]["count"],
                "target range outside the population")
        # the synapse states live in the rows of one pathway: the first on_pre pathway whose program
        # touches them, else the first; on_post and synapse codes use its rows, and the other
        # pathways touching them reach its records through a row map
        state_names = {st[0] for st in syn_states}
        touch = [bool((_reads(code_of[pw["name"]]) | set(code_of[pw["name"]]["effects"]["writes"])) & state_names)
                 for pw in pres]
        owner_position = touch.index(True) if any(touch) else 0
        sharers = []
        for position, pw in enumerate(pres):
            pw_delays = delays if position == 0 else np.asarray(pw["delay_ticks"], np.int64)
            require(pw_delays.size in (1, edge_count), "delay array length")
            pending = _pending_events(pw, spop.start_tick, spop.steps, sdef["source_count"], edge_count, pw_delays)
            dvals = sorted({int(v) for v in pw_delays.tolist()}, reverse=True) if pw_delays.size else [0]
            pathways.append(PathwayPlan(
                index=len(pathways), synapse=s, name=pw["name"], code=code_of[pw["name"]],
                source=sdef["source_population"], target=sdef["target_population"],
                sstart=sdef["source_start"], scount=sdef["source_count"], tstart=sdef["target_start"],
                tcount=sdef["target_count"], topology=topology, edge_count=edge_count, delays=pw_delays, dvals=dvals,
                edge_params=edge_params, scalar_params=scalar_params,
                syn_states=syn_states if position == owner_position or touch[position] else [],
                post_aliases=dict(sdef["post_state_aliases"]), pending=pending, edge_gen=edge_gen,
                random=draws_random(sdef["code_objects"]), event=pw["event"]))
            if position == owner_position:
                owner = pathways[-1]
            elif touch[position]:
                sharers.append(pathways[-1])
        for path in sharers:
            path.state_owner = owner
        synapse_codes += _synapse_code_plans(d, s, sdef, other_codes, owner, populations)
        if post_pathway is not None:
            require(topology[0] == "explicit", "on_post pathways need an explicit topology")
            post_ticks = (prepared_delays[1] if prepared_delays is not None
                          else np.asarray(post_pathway["delay_ticks"], np.int64))
            post_delays = sorted({int(v) for v in post_ticks.tolist()}, reverse=True)
            require(len(post_delays) >= 1 and post_ticks.size in (1, edge_count), "on_post delay array length")
            tpop_ = populations[sdef["target_population"]]
            post_pending = _pending_events(post_pathway, tpop_.start_tick, tpop_.steps, sdef["target_count"],
                                           edge_count, post_ticks)
            if post_pending is not None:
                ticks_, items_, uniform_ = post_pending
                # items are target neurons for a uniform delay, edges otherwise; a tick's events
                # run at once, so none may repeat
                width = sdef["target_count"] if uniform_ else edge_count
                require(np.unique(ticks_ * width + items_).size == items_.size,
                        "pending on_post events repeat a neuron or an edge within one tick")
            post_paths.append(PostPlan(index=-1, synapse=s, name=post_pathway["name"], code=code_of[post_pathway["name"]],
                                       pre=owner, delay=post_delays[0], pending=post_pending,
                                       event=post_pathway["event"], dvals=post_delays,
                                       delays=post_ticks if len(post_delays) > 1 else None))
    _check_pathway_programs(d, pathways)
    _check_post_programs(d, post_paths)
    for post in post_paths:
        written = {w for code in populations[post.pre.target].poisson_inputs for w in code["effects"]["writes"]}
        reads = {post.pre.post_aliases[a] for a in _reads(post.code) if a in post.pre.post_aliases}
        require(not written & reads, "on_post programs reading a state a PoissonInput writes are not supported")
    order, post_order, code_order = _check_schedule(d, populations, pathways, post_paths, synapse_codes)
    pathways = [pathways[k] for k in order]
    post_paths = [post_paths[k] for k in post_order]
    synapse_codes = [synapse_codes[k] for k in code_order]
    for position, path in enumerate(pathways):
        path.index = position
    for position, post in enumerate(post_paths):
        post.index = len(pathways) + position
    split = any(0 in path.dvals for path in pathways)
    for pop in populations:
        for code, where in pop.regular:
            # before the update, not_refractory still holds the previous tick's value, which the
            # kernel does not keep
            require(not (where == "pre" and "not_refractory" in _reads(code)),
                    "run_regularly code reading not_refractory before the update is not supported")
    # with a delay-0 pathway a launch delivers the previous tick, then updates this one: a
    # block may publish this tick's spikes while another still reads the oldest slot the
    # previous tick's deliveries need, so the ring holds one more tick
    extra = 1 if split else 0
    for path in pathways:
        src = populations[path.source]
        # a persistent launch (one population of a size it takes, no delay-0 pathway) lets a
        # workgroup run up to d ticks ahead of a slower one (its deliveries wait for the spikes
        # of tick - d only) and publish tick + d + 1 while the slower one reads tick - d: 2 d + 2
        # slots
        may_persist = (len(populations) == 1 and not synapse_codes and
                       PERSISTENT_MIN_BLOCKS <= src.blocks <= RESIDENT_BLOCKS * 512 // shape.wg)
        ahead = max(path.dvals) + 1 if may_persist else 0
        if path.event != "spike":
            # a custom event's fired neurons go to a ring of their own, published with the spikes
            k = next(k for k, (event, _, _) in enumerate(src.custom_events) if event == path.event)
            src.event_rings[k] = max(src.event_rings.get(k, 1), max(path.dvals) + 1 + extra + ahead)
        else:
            src.ring = max(src.ring, max(path.dvals) + 1 + extra + ahead)
        require(populations[path.source].blocks <= PATH_MAX_SOURCE_BLOCKS, "source population too large")
    for post in post_paths:
        tgt = populations[post.pre.target]
        if post.event != "spike":
            k = next(k for k, (event, _, _) in enumerate(tgt.custom_events) if event == post.event)
            tgt.event_rings[k] = max(tgt.event_rings.get(k, 1), post.delay + 1 + extra)
        else:
            tgt.ring = max(tgt.ring, post.delay + 1 + extra)
    if multi:
        # several clocks: the run is the reference's merged step sequence (executor.rs:3940-3964);
        # a launch per step reads which clocks it advances, and their ticks, from a table
        # a refractory deadline counts its own population's ticks
        require(all("\0not_refractory" not in _touched_post(path)[0] for path in pathways
                    if populations[path.source].clock != populations[path.target].clock),
                "a pathway reading not_refractory across clocks is not supported")
        clock_table = merged_clock_steps(clocks)
        dt, start_tick, steps = clocks[0][0], 0, int(clock_table.shape[0])
    else:
        clock_table = None
        dt, start_tick, steps = clocks[0]
    plan = Plan(document=doc, populations=populations, pathways=pathways, synapse_count=len(d["synapses"]),
                synapse_edges=synapse_edges, dt=dt, start_tick=start_tick, steps=steps, split=split, shape=shape,
                post_paths=post_paths, synapse_codes=synapse_codes, clock_table=clock_table, clocks=clocks)
    plan.total_blocks = first_block
    plan.rng_seed = int(inst.get("rng_seed", 0))
    return plan


def _synapse_code_plans(d: dict, s: int, sdef: dict, codes: list, path: PathwayPlan, populations: list) -> list:
    """The clock-driven state update and summed variables of one Synapses, checked as
    model.rs:4394-4500 checks their metadata (one state update for a non-empty, duplicate-free
    clock-driven state list, writing only those states; a summed variable into one floating-point
    state of its endpoint population, with no pathway metadata).  Their programs here read the
    edge's synapse states and parameters, the endpoint indices and, for a summed variable, the
    target's states; each runs in the groups slot."""
    clock_driven = list(sdef.get("clock_driven_states", []))
    syn_names = {st[0] for st in path.syn_states}
    require(len(set(clock_driven)) == len(clock_driven) and set(clock_driven) <= syn_names,
            "invalid clock-driven synaptic state list")
    require(sum(c["kind"] == "synapse_state_update" for c in codes) == (1 if clock_driven else 0),
            "expected one synapse state update for the clock-driven states")
    pre_aliases = set(sdef["pre_state_aliases"])
    out = []
    for code in codes:
        kind = code["kind"]
        require(kind in ("synapse_state_update", "summed_variable"), f"synapse code object kind {kind!r} is not supported")
        require(code.get("when") == "groups", f"a {kind} runs in the groups slot here")
        require(code.get("adaptive") is None, "adaptive integrators are not supported")
        require(code.get("pathway_name") is None, f"pathway metadata on a {kind} code object")
        reads = _reads(code)
        require(not reads & (pre_aliases | {"i", "not_refractory_post", "lastspike_post", "not_refractory"}),
                f"{kind} programs reading the source population or refractoriness are not supported")
        if kind == "synapse_state_update":
            # it reads no neuron state, so it commutes with every population node of the slot
            require(not reads & set(path.post_aliases), "synapse state updates reading neuron state are not supported")
            require(set(code["effects"]["writes"]) <= set(clock_driven),
                    "a synapse state update writes clock-driven states only")
            out.append(SynCodePlan(kind="update", synapse=s, code=code, path=path))
            continue
        target = code.get("summed_target")
        require(target in ("pre", "post"), "invalid summed variable endpoint")
        to_pre = target == "pre"
        population = sdef["source_population"] if to_pre else sdef["target_population"]
        pop = populations[population]
        dtype = next((st[1] for st in pop.states if st[0] == code.get("summed_state")), None)
        require(dtype in ("f32", "f64"), "summed variable target must be floating-point population state")
        state = code["summed_state"]
        require(not code["effects"]["writes"], "a summed variable program writes no state")
        require(any(st["target"] == "_synaptic_var" for st in code["vector"]), "missing summed expression result")
        # the summed state is zeroed and accumulated over the edges: a program reading it would
        # see the partial sum
        require(not (to_pre and reads & set(path.post_aliases)),
                "summed variables into the source population reading target state are not supported")
        require(not any(path.post_aliases[a] == state for a in reads if a in path.post_aliases)
                or population != path.target, "a summed variable reading its own target state is not supported")
        require(not (pop.monitor_record and state in pop.monitor_vars),
                "a state monitor recording a summed variable's state is not supported")
        out.append(SynCodePlan(kind="summed", synapse=s, code=code, path=path, to_pre=to_pre, state=state,
                               dtype=dtype, population=population,
                               start=sdef["source_start"] if to_pre else sdef["target_start"],
                               count=sdef["source_count"] if to_pre else sdef["target_count"]))
    return out


def merged_clock_steps(clocks: list) -> np.ndarray:
    """The reference's merged step sequence of several clocks (Runtime::advance, executor.rs:
    3940-3964): each step advances every clock whose next tick time lies within epsilon (the
    smallest dt times 1e-12) of the earliest next tick time among the clocks not yet at their end.
    Returns int64 [steps, clocks]: each clock's tick at that step, -1 where it does not advance."""
    epsilon = min(dt for dt, _, _ in clocks) * 1e-12
    ticks = [start for _, start, _ in clocks]
    ends = [start + count for _, start, count in clocks]
    rows = []
    while True:
        pending = [ticks[c] * clocks[c][0] for c in range(len(clocks)) if ticks[c] < ends[c]]
        if not pending:
            break
        now = min(pending)
        active = [ticks[c] < ends[c] and abs(ticks[c] * clocks[c][0] - now) <= epsilon for c in range(len(clocks))]
        require(any(active), "no clock advances at the earliest tick time")
        rows.append([ticks[c] if active[c] else -1 for c in range(len(clocks))])
        for c in range(len(clocks)):
            ticks[c] += int(active[c])
    return np.asarray(rows, np.int64).reshape(-1, len(clocks))


def _binary_csr(sdef: dict, sin: dict) -> tuple[np.ndarray, np.ndarray, dict]:
    """Edges of a ``binary_csr`` topology (a B2CSR001 file): source and target indices in
    file order and each per-edge parameter's column.  The declaration is checked as
    model.rs:2163-2204 does (no inline edges or synapse states, every per-edge parameter
    f64 and mapped to one column, the columns used once each, a SHA-256 digest, on_pre
    pathways of one uniform delay), the file as binary_topology.rs:24-130 does.  A relative
    path is taken from the working directory, as the reference opens it."""
    from . import binary_topology
    topo = sin["topology"]
    per_edge = [p for p in sdef["parameters"] if p["index_domain"] == "synapse"]
    initializers = {name: int(column) for name, column in topo["initializers"].items()}
    sha = str(topo["sha256"])
    require(not sin.get("source") and not sin.get("target") and not sdef["states"]
            and all(p["dtype"] == "f64" for p in per_edge)
            and {p["name"] for p in per_edge} == set(initializers)
            and sorted(initializers.values()) == list(range(int(topo["column_count"])))
            and len(sha) == 64 and all(c in "0123456789abcdefABCDEF" for c in sha)
            and all(pw["kind"] == "pre" and pw.get("delay_initializer") is None and len(pw["delay"]) == 1
                    for pw in sin["pathways"]), "invalid binary CSR mapping/pathway")
    try:
        src, tgt, values = binary_topology.read_csr(topo["path"], sdef["source_count"], sdef["target_count"],
                                                    int(topo["edge_count"]), int(topo["column_count"]), sha)
    except (OSError, binary_topology.BinaryCsrError) as error:
        raise UnsupportedModel(str(error)) from error
    return src, tgt, {name: values[column] for name, column in initializers.items()}


def _pending_events(pw: dict, start_tick: int, steps: int, endpoints: int, edges: int,
                    delays: np.ndarray) -> tuple | None:
    """A pathway's pending events (a continuation's), checked as model.rs:4322-4338 does
    (delivery ticks ascending and inside the endpoint's run, items endpoints for a uniform
    delay and edges otherwise), as (tick offset from the run start, item, uniform).  The
    reference files an event into queue slot delivery_tick % L, L = min(largest delay + 1,
    steps) (executor.rs:6185-6205), so it is delivered at the run's first tick of that slot."""
    events = pw.get("pending") or []
    if not events:
        return None
    ticks = np.fromiter((int(e["delivery_tick"]) for e in events), np.int64, len(events))
    items = np.fromiter((int(e["item"]) for e in events), np.int64, len(events))
    uniform = delays.size > 0 and bool(np.all(delays == delays[0]))
    limit = endpoints if uniform else edges
    require(len(events) <= 10_000_000 and bool(np.all(np.diff(ticks) >= 0))
            and bool(np.all((ticks >= start_tick) & (ticks < start_tick + steps)))
            and bool(np.all((items >= 0) & (items < limit))), "invalid pending synaptic pathway event")
    length = min(int(delays.max(initial=0)) + 1, steps)
    return (ticks - start_tick) % length, items, uniform


def pending_layout(plan: "Plan", group: list[PathwayPlan]) -> tuple[np.ndarray, np.ndarray, int]:
    """The pending events of a delivery group per (tick offset, target block): offsets
    u32[T * TB + 1] and entries u32[n, 2] = (row, block-local target | pathway << 16), and
    T, the ticks covered.  A uniform-delay event is its source's out-edges, edges ascending
    (executor.rs:2345-2380); each pathway's events keep the order given."""
    block = plan.shape.block
    TB = plan.populations[group[0].target].blocks
    ks, targets, rows, paths = [], [], [], []
    for p, path in enumerate(group):
        if path.pending is None:
            continue
        offs, items, uniform = path.pending
        _, src, tgt = path.topology
        row_of_edge = np.empty(path.edge_count, np.int64)
        row_of_edge[path.order] = np.arange(path.edge_count, dtype=np.int64)
        if uniform:
            by_source = np.argsort(src, kind="stable")
            ordered = src[by_source]
            first = np.searchsorted(ordered, items, "left")
            n = np.searchsorted(ordered, items, "right") - first
            event = np.repeat(np.arange(items.size), n)
            within = np.arange(event.size) - np.repeat(np.cumsum(n) - n, n)
            edges, k = by_source[first[event] + within], offs[event]
        else:
            edges, k = items, offs
        if not counting_group(group):
            # staged events of one flush run their per-edge statements at once
            require(np.unique(k * path.edge_count + row_of_edge[edges]).size == edges.size,
                    "pending events repeat an edge within one tick")
        ks.append(k)
        targets.append(np.asarray(tgt, np.int64)[edges] + path.tstart)
        rows.append(row_of_edge[edges])
        paths.append(np.full(edges.size, p, np.int64))
    k, target, row, path_ = (np.concatenate(a) for a in (ks, targets, rows, paths))
    blocks = target // block
    order = np.lexsort((np.arange(k.size), blocks, k))
    ticks = int(k.max(initial=0)) + 1
    offsets = np.zeros(ticks * TB + 1, np.int64)
    np.cumsum(np.bincount(k * TB + blocks, minlength=ticks * TB), out=offsets[1:])
    entries = np.stack([row[order], (target[order] % block) | (path_[order] << 16)], axis=1)
    return offsets.astype(np.uint32), entries.astype(np.uint32), ticks


def pending_as_sources(plan: "Plan", group: list[PathwayPlan]) -> bool:
    """A counting group of one delay delivered by pull takes its pending events as pending
    sources (uniform delays: an event is its source's out-edges, executor.rs:2345-2362): the
    tick's list of source ids runs through the same segment lookup as the fired ones, so the
    host needs no edge of a procedural topology."""
    return (counting_group(group) and not push_group(plan, group) and group[0].index not in plan.queues
            and len({d for path in group for d in path.dvals}) == 1
            and all(path.pending is None or path.pending[2] for path in group))


def pending_source_layout(plan: "Plan", group: list[PathwayPlan]) -> tuple[np.ndarray, np.ndarray, int] | None:
    """Pending sources of a counting group per tick offset: offsets u32[T + 1] and source-
    population ids.  A listed id counts for every pathway of the group whose source range
    holds it, so each tick's list must give each pathway exactly its own pending sources
    (the same multiset; counting makes their order free).  None when it cannot (pathways
    whose source ranges overlap, with different pending sources)."""
    by_tick: dict = {}
    for path in group:
        if path.pending is not None:
            k, items, _ = path.pending
            for tick, item in zip(k.tolist(), items.tolist()):
                by_tick.setdefault(tick, []).append(item + path.sstart)
    ticks = max(by_tick) + 1 if by_tick else 1
    for tick, ids in by_tick.items():
        listed = np.asarray(ids, np.int64)
        for path in group:
            mine = np.sort(listed[(listed >= path.sstart) & (listed < path.sstart + path.scount)] - path.sstart)
            own = np.sort(path.pending[1][path.pending[0] == tick]) if path.pending is not None else np.zeros(0)
            if not np.array_equal(mine, own):
                return None
    offsets = np.zeros(ticks + 1, np.int64)
    np.cumsum([len(by_tick.get(t, [])) for t in range(ticks)], out=offsets[1:])
    ids = np.asarray([v for t in range(ticks) for v in by_tick.get(t, [])], np.int64)
    return offsets.astype(np.uint32), ids.astype(np.uint32), ticks


def post_pending_layout(plan: "Plan", post: PostPlan) -> tuple[np.ndarray, np.ndarray, int]:
    """Pending on_post events per (tick offset, block of the target population): offsets
    u32[T * NB + 1] and the population indices of the neurons whose events arrive (u32; with
    per-edge delays the rows of the edges whose events arrive), in the order given, and T."""
    block = plan.shape.block
    NB = plan.populations[post.pre.target].blocks
    k, items, uniform = post.pending
    if uniform:
        ids = items + post.pre.tstart
        blocks = ids // block
    else:
        # per-edge delays: the items are edges, listed as their rows (the target's block runs them)
        pre = post.pre
        row_of_edge = np.empty(pre.edge_count, np.int64)
        row_of_edge[pre.order] = np.arange(pre.edge_count, dtype=np.int64)
        blocks = (np.asarray(pre.topology[2], np.int64)[items] + pre.tstart) // block
        ids = row_of_edge[items]
    order = np.lexsort((np.arange(k.size), blocks, k))
    ticks = int(k.max(initial=0)) + 1
    offsets = np.zeros(ticks * NB + 1, np.int64)
    np.cumsum(np.bincount(k * NB + blocks, minlength=ticks * NB), out=offsets[1:])
    return offsets.astype(np.uint32), ids[order].astype(np.uint32), ticks


EVENT_MONITOR_BUDGET = 10_000_000   # events one EventMonitor may record (executor.rs:3061-3066)


def spike_generator_schedule(spec: dict, count: int, start_tick: int, steps: int) -> tuple[np.ndarray, np.ndarray]:
    """A SpikeGeneratorGroup's (tick, neuron) schedule (model.rs:3762-3790: strictly increasing
    pairs, ticks inside the run, neurons inside the group; executor.rs:3008-3036 emits, at each
    tick, the neurons scheduled for it in ascending order) regrouped per neuron: offsets
    u32[count + 1] and each neuron's ticks ascending (u32), so a neuron's update needs one
    cursor and one load per tick."""
    ticks = np.asarray(spec["spike_ticks"], np.int64)
    neurons = np.asarray(spec["spike_indices"], np.int64)
    require(ticks.size == neurons.size and ticks.size <= 10_000_000, "invalid SpikeGeneratorGroup schedule")
    if ticks.size:
        require(bool(np.all((ticks >= start_tick) & (ticks < start_tick + steps) & (neurons >= 0) & (neurons < count))),
                "invalid SpikeGeneratorGroup schedule")
        pairs = ticks * count + neurons
        require(bool(np.all(np.diff(pairs) > 0)), "invalid SpikeGeneratorGroup schedule")
        require(int(ticks.max()) < 2**32, "spike ticks beyond u32")
    order = np.lexsort((ticks, neurons))
    offsets = np.zeros(count + 1, np.uint32)
    np.cumsum(np.bincount(neurons, minlength=count), out=offsets[1:])
    return offsets, ticks[order].astype(np.uint32)


def _reads(code: dict) -> set:
    out: set = set()

    def walk(e):
        if isinstance(e, dict):
            if e.get("op") == "load":
                out.add(e["name"])
            for v in e.values():
                walk(v)
        elif isinstance(e, list):
            for v in e:
                walk(v)
    for st in code["scalar"] + code["vector"]:
        walk(st["value"])
        if st.get("condition"):
            out.add(st["condition"])
    return out


def _check_pathway_programs(d: dict, pathways: list) -> None:
    for path in pathways:
        sdef = d["synapses"][path.synapse]
        reads = _reads(path.code)
        pre = set(sdef["pre_state_aliases"])
        require(not (reads & pre), "pathway programs reading presynaptic state are not supported")
        require("i" not in reads, "pathway programs reading the source index are not supported")
        for name in path.code["effects"]["writes"]:
            require(name in path.post_aliases or name in {s[0] for s in path.syn_states},
                    f"pathway write to {name!r} is not supported")


def _check_post_programs(d: dict, post_paths: list) -> None:
    for post in post_paths:
        sdef = d["synapses"][post.synapse]
        reads = _reads(post.code)
        neuron = set(sdef["pre_state_aliases"]) | set(sdef["post_state_aliases"]) | {"i", "j", "not_refractory_post"}
        require(not (reads & neuron), "on_post programs reading neuron state are not supported")
        for name in post.code["effects"]["writes"]:
            require(name in {s_[0] for s_ in post.pre.syn_states}, f"on_post write to {name!r} is not supported")


def _check_schedule(d: dict, populations: list, pathways: list, post_paths: list,
                    synapse_codes: list = ()) -> tuple[list, list, list]:
    """The per-tick node order must match the fused phase order (monitors, summed variables,
    update, threshold, every on_pre pathway, every on_post pathway, reset); returns the pre
    and post pathway orders and the order of the synapse codes run before the tick kernel.  A
    synapse state update reads only its synapse's states and parameters, so it commutes with
    every population node and keeps only its place among the synapse codes."""
    nodes = d["schedule"]["nodes"]
    require(nodes, "an empty schedule uses the legacy phase loop")
    slots = d["schedule"]["slots"]
    rank = {name: position for position, name in enumerate(slots)}
    phase_of = []
    path_order, post_order = [], []
    by_pathway = {(path.synapse, path.name): k for k, path in enumerate(pathways)}
    post_by_synapse = {post.synapse: k for k, post in enumerate(post_paths)}
    code_by_id = {id(c.code): k for k, c in enumerate(synapse_codes)}
    code_order = []
    poisson_nodes: dict = {}
    regular_places: dict = {}
    reset_orders: dict = {}
    for node in nodes:
        op, owner = node["operation"], node["owner_kind"]
        if owner == "population":
            pop = d["populations"][node["owner_index"]]
            require(node["clock"] == pop["clock"], "a population's schedule nodes run on its clock")
            if op == "state_monitor":
                phase = 0
            elif op in ("spike_monitor", "event_source"):
                phase = 2
            elif op == "event_monitor":
                # at the thresholds slot it records at the threshold, before any delivery or reset
                # (after its event's threshold node); at the end slot after the resets
                monitor = pop["event_monitors"][node["item_index"]]
                require(any(n["operation"] == "code_object" and n["owner_kind"] == "population" and
                            n["owner_index"] == node["owner_index"] and
                            pop["code_objects"][n["item_index"]]["kind"] == "threshold" and
                            pop["code_objects"][n["item_index"]].get("event_name", "spike") == monitor["event"]
                            for n in nodes[:nodes.index(node)]),
                        "an event monitor must follow its event's threshold")
                phase = 2 if monitor["when"] == "thresholds" else 4.25
            elif op == "code_object":
                kind = pop["code_objects"][node["item_index"]]["kind"]
                if kind == "run_regularly":
                    # before the population's update, between the update and the threshold, or
                    # after the reset (the kernel runs it inside the update or at the tick's end),
                    # by its slot and its place among the population's own nodes
                    own = [(n["item_index"], pop["code_objects"][n["item_index"]]["kind"]) for n in nodes
                           if n["operation"] == "code_object" and n["owner_kind"] == "population"
                           and n["owner_index"] == node["owner_index"]]
                    before = {kind_ for _, kind_ in own[:own.index((node["item_index"], kind))]}
                    when = rank[node["when"]]
                    if when <= rank["groups"] and "state_update" not in before:
                        place, phase = "pre", 0.75
                    elif when <= rank["thresholds"] and "threshold" not in before:
                        place, phase = "mid", 1.5
                    else:
                        require(when >= rank["resets"] and ("reset" in before or
                                                            not any(k_ == "reset" for _, k_ in own)),
                                "run_regularly code between the threshold and the reset is not supported")
                        place, phase = "end", 4.5
                    regular_places[(node["owner_index"], node["item_index"])] = place
                    phase_of.append(phase)
                    continue
                # PoissonInput runs in the synapses slot at order 0 (export.py:607), after the
                # on_pre pathways (order -1) and before the on_post ones (order 1)
                phase = {"state_update": 1, "threshold": 2, "poisson_input": 3.25, "reset": 4}[kind]
                # an event's condition runs in the update's step, its reset in the resets slot
                require(kind not in ("threshold", "reset") or
                        node["when"] == {"threshold": "thresholds", "reset": "resets"}[kind],
                        f"{kind} code outside the {kind}s slot is not supported")
                if kind == "reset":
                    reset_orders.setdefault(node["owner_index"], []).append(
                        pop["code_objects"][node["item_index"]].get("event_name", "spike"))
                if kind == "poisson_input":
                    poisson_nodes.setdefault(node["owner_index"], []).append(node["item_index"])
            else:
                raise UnsupportedModel(f"schedule operation {op!r} is not supported")
        else:
            require(op == "code_object", f"synapse schedule operation {op!r} is not supported")
            sdef = d["synapses"][node["owner_index"]]
            code = sdef["code_objects"][node["item_index"]]
            kind = code["kind"]
            # a pathway runs on the clock of the population whose spikes trigger it, so its delay
            # queue and its spike reads share one tick count
            trigger = {"synapses": "source_population", "synapses_post": "target_population"}.get(kind)
            if trigger is not None:
                require(node["clock"] == d["populations"][sdef[trigger]]["clock"],
                        "a pathway runs on the clock of the population that triggers it")
            else:
                # a summed variable or state update runs when its own clock advances (the synapse
                # code kernel reads its clock's tick from the clock table); a summed variable on the
                # clock of the population whose state it sets
                require(node["clock"] == code.get("clock", node["clock"]),
                        "a synapse code object's schedule node must carry its clock")
                if kind == "summed_variable":
                    endpoint = "target_population" if code.get("summed_target") == "post" else "source_population"
                    require(node["clock"] == d["populations"][sdef[endpoint]]["clock"],
                            "a summed variable runs on the clock of the population it sets")
            if kind == "synapses":
                phase = 3
                path_order.append(by_pathway[(node["owner_index"], code.get("pathway_name"))])
            elif kind == "synapses_post":
                phase = 3.5
                post_order.append(post_by_synapse[node["owner_index"]])
            else:
                code_order.append(code_by_id[id(code)])
                if kind == "synapse_state_update":
                    continue
                phase = 0.5
        phase_of.append(phase)
    require(all(a <= b for a, b in zip(phase_of, phase_of[1:])),
            "schedule order differs from monitor/summed/update/threshold/synapses/reset")
    for index, items in poisson_nodes.items():
        # the kernel runs a population's PoissonInputs in code-object order
        require(items == sorted(items), "PoissonInputs scheduled out of code-object order")
    for p, pop in enumerate(populations):
        # run_regularly code in schedule order, with its place in the tick
        codes = d["populations"][p]["code_objects"]
        pop.regular = [(codes[item], place) for (owner, item), place in regular_places.items() if owner == p]
        pop.reset_order = reset_orders.get(p, [])
        # end-of-tick event monitors record right after the resets, before end-of-tick run_regularly code
        require(not (any(when == "end" for _, _, _, when in pop.event_monitors) and
                     any(place == "end" for _, place in pop.regular)),
                "end-of-tick event monitors with end-of-tick run_regularly code are not supported")
    del rank
    require(len(path_order) == len(pathways) and len(post_order) == len(post_paths)
            and sorted(code_order) == list(range(len(synapse_codes))),
            "every pathway and synapse code object needs one schedule node")
    return path_order, post_order, code_order


# ----------------------------------------------------------------- layouts
def explicit_layout(path: PathwayPlan, target_blocks: int, block_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Source-major rows sorted by (delay group, target block, target, edge).

    Returns (row_target u32, segment u32[(S*D)*(NBT+1)], order edge ids per row).
    """
    _, src, tgt = path.topology
    delays = path.delays if path.delays.size == path.edge_count else np.full(path.edge_count, path.dvals[0])
    group_of = {value: g for g, value in enumerate(path.dvals)}
    lut = np.zeros(max(path.dvals) + 1, np.int64)
    for value, g in group_of.items():
        lut[value] = g
    group = lut[delays] if path.edge_count else np.zeros(0, np.int64)
    tpop = tgt + path.tstart
    block = tpop // block_size
    D, NB, S = len(path.dvals), target_blocks, path.scount
    if S * D * NB * block_size < 2**62:
        # one composite key; the stable sort keeps edge order among equal keys
        composite = ((src * D + group) * NB + block) * block_size + (tpop - block * block_size)
        order = np.argsort(composite, kind="stable")
        del composite
    else:
        order = np.lexsort((np.arange(path.edge_count, dtype=np.int64), tpop, block, group, src))
    key = (src * D + group) * NB + block
    counts = np.bincount(key, minlength=S * D * NB).reshape(S * D, NB)
    row_start = np.zeros(S * D + 1, np.int64)
    np.cumsum(counts.sum(axis=1), out=row_start[1:])
    seg = np.empty((S * D, NB + 1), np.int64)
    seg[:, 0] = row_start[:-1]
    np.cumsum(counts, axis=1, out=seg[:, 1:])
    seg[:, 1:] += row_start[:-1, None]
    require(path.edge_count < 2**32, "edge count beyond u32")
    return tpop[order].astype(np.uint32), seg.reshape(-1).astype(np.uint32), order


def post_major_layout(path: PathwayPlan, target_blocks: int, block_size: int) -> tuple[np.ndarray, ...]:
    """Rows ordered by (target, source, delay group, edge): the incoming edges of a target are
    one run of consecutive rows, so an on_post pass over a spiking neuron's edges reads and writes
    its synapse records as one contiguous range.  Within a target, rows keep the order of the
    source-major layout (source, delay group, edge), which the canonical delivery order of
    queued events compares.  The segment and target tables stay source-major, over out-edge
    positions; out_row maps a position to its row.

    Returns (target per position u32, segment u32[(S*D)*(NBT+1)], order edge ids per row,
    out_row u32 per position)."""
    out_tgt, seg, out_order = explicit_layout(path, target_blocks, block_size)
    _, src, tgt = path.topology
    delays = path.delays if path.delays.size == path.edge_count else np.full(path.edge_count, path.dvals[0])
    lut = np.zeros(max(path.dvals) + 1, np.int64)
    for g, value in enumerate(path.dvals):
        lut[value] = g
    group = lut[delays] if path.edge_count else np.zeros(0, np.int64)
    src = np.asarray(src, np.int64)
    tpop = np.asarray(tgt, np.int64) + path.tstart
    D = len(path.dvals)
    order = np.argsort((tpop * path.scount + src) * D + group, kind="stable")
    row_of_edge = np.empty(path.edge_count, np.int64)
    row_of_edge[order] = np.arange(path.edge_count, dtype=np.int64)
    return out_tgt, seg, order, row_of_edge[out_order].astype(np.uint32)


def post_major_paths(plan: "Plan") -> set:
    """Pathways whose rows are ordered by target: explicit pre pathways of an on_post pathway,
    with synapse states, delivered as a queued group (whose pushes look the out-edges up by
    position, and whose events carry their row)."""
    pres = {post.pre.index for post in plan.post_paths}
    out = set()
    for group in delivery_groups(plan):
        if queue_limits(plan, group) is None:
            continue
        for path in group:
            if path.index in pres and path.topology[0] == "explicit" and path.syn_states and path.edge_count:
                out.add(path.index)
    return out


def initial_until(lastspike: np.ndarray, start_tick: int, dt: float, period: int) -> np.ndarray:
    """First tick >= start at which the fixed-refractory recompute yields true.

    ``not_refractory = timestep(tick*dt - lastspike, dt) >= period`` (executor.rs:
    4045-4058, model.rs:981-992) is monotone in the tick, so it is true exactly
    from this tick on.  Evaluated with the same f64 operations as the device.
    """
    def available(tick: int, last: float) -> bool:
        steps = (tick * dt - last + 1e-3 * dt) / dt
        require(tick * dt - last >= 0.0, "initial lastspike lies after the run start")
        return int(steps) >= period
    out = np.empty(lastspike.size, np.int32)
    cache: dict[float, int] = {}
    for k, last in enumerate(lastspike.tolist()):
        if last not in cache:
            c = start_tick
            if not available(c, last):
                c = max(start_tick, int(math.floor(last / dt)) + period - 2)
                while not available(c, last):
                    c += 1
                while c - 1 >= start_tick and available(c - 1, last):
                    c -= 1
            require(c < 2**31 - 1, "refractory tick beyond the i32 range")
            cache[last] = c
        out[k] = cache[last]
    return out


UNTIL_TABLE_TICKS = 1 << 24   # longest run whose refractory deadlines are tabulated (4 bytes per tick)


def refractory_table(start_tick: int, steps: int, dt_clock: float, dt: float, period: int) -> np.ndarray | None:
    """The refractory deadline of a spike at each tick of the run, as the device's
    refractory_until computes it (atlas_tick.h): the first tick c > tick whose recompute
    ``timestep(c dt_clock - tick dt_clock, dt) >= period`` holds (executor.rs:4045-4058), searched
    from tick + period, 8 steps down then 8 up, with the same f64 operations.  Fixed
    refractoriness with one period makes it a function of the tick alone, so a launch reads it
    instead of dividing per spike.  None when a search would fault (the device then searches
    itself and reports it at the tick a neuron fires) or the run is longer than
    UNTIL_TABLE_TICKS."""
    if steps <= 0 or steps > UNTIL_TABLE_TICKS:
        return None
    tick = np.arange(start_tick, start_tick + steps, dtype=np.int64)
    t = tick.astype(np.float64) * dt_clock
    eps = 1e-3 * dt
    faulted = np.zeros(steps, bool)

    def timestep(c, evaluated):
        nonlocal faulted
        time = c.astype(np.float64) * dt_clock - t
        with np.errstate(all="ignore"):
            steps_ = (time + eps) / dt
        ok = (time >= 0.0) & (steps_ < 9223372036854775808.0)
        faulted |= evaluated & ~ok
        return np.where(ok, np.trunc(np.where(ok, steps_, 0.0)), 0.0).astype(np.int64)

    c = tick + period
    c = np.where(c <= tick, tick + 1, c)
    for _ in range(8):
        below = c - 1 > tick
        move = below & (timestep(c - 1, below) >= period)
        if not move.any():
            break
        c = c - move
    for _ in range(8):
        move = timestep(c, np.ones(steps, bool)) < period
        if not move.any():
            break
        c = c + move
    at = timestep(c, np.ones(steps, bool))
    check = (at >= period) & (c - 1 > tick)
    faulted |= (at < period) | (check & (timestep(c - 1, check) >= period))
    if faulted.any() or c.max() >= 2**31 - 1:
        return None
    return c.astype(np.int32)


# ------------------------------------------------------------------ codegen
def _monitor_entries(pop: PopulationPlan, block_size: int) -> tuple[np.ndarray, np.ndarray]:
    record = np.asarray(pop.monitor_record, np.int64)
    blocks = record // block_size
    order = np.argsort(blocks, kind="stable")
    entries = np.stack([order, record[order]], axis=1).astype(np.uint32).reshape(-1)
    offsets = np.zeros(pop.blocks + 1, np.uint32)
    np.cumsum(np.bincount(blocks, minlength=pop.blocks), out=offsets[1:])
    return entries, offsets


def allocate(plan: Plan) -> None:
    """Assign device buffers (table indices) for every array the module touches."""
    plan.buffers.clear()
    plan.fault_buffer = plan.add("fault", 16)
    if plan.clock_table is not None:
        plan.clock_buffer = plan.add("clock_table", plan.clock_table.nbytes, plan.clock_table)
    for pop in plan.populations:
        b = pop.buffers
        for name, dtype, values in pop.states:
            b[f"state:{name}"] = plan.add(f"p{pop.index}.{name}", values.nbytes, values)
        for name, (dtype, values) in pop.vector_params.items():
            b[f"param:{name}"] = plan.add(f"p{pop.index}.param.{name}", values.nbytes, values.astype(np.float64))
        if pop.refractory is not None:
            _, lastspike, _, until = pop.refractory
            b["lastspike"] = plan.add(f"p{pop.index}.lastspike", lastspike.nbytes, lastspike.astype(np.float64))
            b["until"] = plan.add(f"p{pop.index}.refractory_until", until.nbytes, until)
            table = refractory_table(pop.start_tick, pop.steps, pop.dt, pop.dt, pop.refractory[0])
            if table is not None:
                b["until_table"] = plan.add(f"p{pop.index}.refractory_table", table.nbytes, table)
        if pop.generator is not None:
            offsets, ticks = pop.generator
            b["gen_offsets"] = plan.add(f"p{pop.index}.generator_offsets", offsets.nbytes, offsets)
            b["gen_ticks"] = plan.add(f"p{pop.index}.generator_ticks", max(4, ticks.nbytes), ticks if ticks.size else None)
            b["gen_cursor"] = plan.add(f"p{pop.index}.generator_cursor", offsets.nbytes - 4, offsets[:-1].copy())
        for k, (_, variables, _, _) in enumerate(pop.event_monitors):
            # records (tick, neuron, values as f64) appended at the threshold; the counter may pass
            # the capacity (the host then reports the budget exceeded)
            b[f"emon_count:{k}"] = plan.add(f"p{pop.index}.event_monitor{k}.count", 8)
            b[f"emon:{k}"] = plan.add(f"p{pop.index}.event_monitor{k}.records",
                                      max(8, pop.event_monitor_capacity(k) * 8 * (1 + len(variables))))
        b["spk_cnt"] = plan.add(f"p{pop.index}.spike_counts", pop.ring * pop.blocks * 4)
        b["spk_small"] = plan.add(f"p{pop.index}.spike_first_ids", pop.ring * pop.blocks * 32)
        b["spk_ids"] = plan.add(f"p{pop.index}.spike_ids", pop.ring * pop.count * 4)
        rows = pop.start_tick + pop.steps - pop.window_start
        pop.buffers["rec_words"] = (pop.count + 31) // 32
        if pop.has_spike_event:
            b["rec"] = plan.add(f"p{pop.index}.spike_bitmap", rows * pop.buffers["rec_words"] * 4)
        for k, _ in enumerate(pop.custom_events):
            # a custom event's flag per neuron (written at the threshold, read by the resets slot
            # of the same tick) and its stream as a bitmap per tick of the recording window
            b[f"evt:{k}"] = plan.add(f"p{pop.index}.event{k}.flags", pop.count)
            b[f"evrec:{k}"] = plan.add(f"p{pop.index}.event{k}.bitmap", max(4, rows * pop.buffers["rec_words"] * 4))
        for k, ring in pop.event_rings.items():
            # the spike ring's layout: counts per (slot, block), ids per slot, the first 8 ids per block
            b[f"ering_cnt:{k}"] = plan.add(f"p{pop.index}.event{k}.ring_counts", ring * pop.blocks * 4)
            b[f"ering_ids:{k}"] = plan.add(f"p{pop.index}.event{k}.ring_ids", ring * pop.count * 4)
            b[f"ering_small:{k}"] = plan.add(f"p{pop.index}.event{k}.ring_small", ring * pop.blocks * 8 * 4)
        if pop.monitor_record and pop.monitor_vars:
            entries, offsets = _monitor_entries(pop, plan.shape.block)
            b["mon_entries"] = plan.add(f"p{pop.index}.monitor_entries", entries.nbytes, entries)
            b["mon_offsets"] = plan.add(f"p{pop.index}.monitor_offsets", offsets.nbytes, offsets)
            for name in pop.monitor_vars:
                dtype = _var_dtype(pop, name)
                b[f"sample:{name}"] = plan.add(f"p{pop.index}.samples.{name}",
                                               rows * len(pop.monitor_record) * np.dtype(NUMPY[dtype]).itemsize)
    plan.delivered_buffer = plan.add("delivered", max(1, len(plan.pathways) + len(plan.post_paths)) *
                                     plan.total_blocks * 8)
    # grid-barrier counters of persistent launches (atlas_tick.h grid_arrive: 2 max delay + 2
    # slots of 32 counters, 64 B apart), zeroed before each launch
    slots = 2 * max([max(path.dvals) for path in plan.pathways] + [0]) + 2
    plan.barrier_buffer = plan.add("grid_barrier", slots * 32 * 64)
    post_major = post_major_paths(plan)
    for path in plan.pathways:
        b = path.buffers
        tpop = plan.populations[path.target]
        NB = tpop.blocks
        D = len(path.dvals)
        if path.topology[0] == "explicit":
            path.post_major = path.index in post_major
            if path.post_major:
                row_tgt, seg, order, out_row = post_major_layout(path, NB, plan.shape.block)
                b["out_row"] = plan.add(f"path{path.index}.out_row", out_row.nbytes, out_row)
                if any(code.path is path for code in plan.synapse_codes):
                    # the target of every row, for the index j of synapse codes
                    by_row = (np.asarray(path.topology[2], np.int64)[order] + path.tstart).astype(np.uint32)
                    b["row_tgt_rows"] = plan.add(f"path{path.index}.row_target_by_row", by_row.nbytes, by_row)
            else:
                row_tgt, seg, order = explicit_layout(path, NB, plan.shape.block)
            path.order = order
            b["row_tgt"] = plan.add(f"path{path.index}.row_target", max(4, row_tgt.nbytes), row_tgt if row_tgt.size else None)
            b["seg"] = plan.add(f"path{path.index}.segment", seg.nbytes, seg)
            if path.random:
                # the edge index of every row, for the counter RNG of the projection's programs
                ids = order.astype(np.uint32)
                b["edge_id"] = plan.add(f"path{path.index}.edge_id", max(4, ids.nbytes), ids if ids.size else None)
        else:
            require(D == 1, "procedural projections need a uniform delay")
            b["row_tgt"] = plan.add(f"path{path.index}.row_target", path.edge_count * 4)
            b["seg"] = plan.add(f"path{path.index}.segment", path.scount * (NB + 1) * 4)
            path.order = None
        for name, (dtype, values) in path.edge_params.items():
            if values is None:   # generated where read
                continue
            row_values = values[path.order] if path.order is not None else values
            b[f"eparam:{name}"] = plan.add(f"path{path.index}.param.{name}", row_values.nbytes,
                                           row_values.astype(np.float64))
        if path.syn_states and path.state_owner is None:
            # the synapse states of a row in one record (widest first, the stride a power of
            # two): an event reads and writes one cache line of them, not one per state
            layout = sorted(path.syn_states, key=lambda st: -np.dtype(NUMPY[st[1]]).itemsize)
            offset = 0
            for name, dtype, _ in layout:
                path.syn_fields[name] = (offset, dtype)
                offset += np.dtype(NUMPY[dtype]).itemsize
            path.syn_stride = 1 << max(2, (offset - 1).bit_length())
            records = np.zeros(path.edge_count, syn_record_dtype(path))
            for name, dtype, values in path.syn_states:
                records[name] = values[path.order] if path.order is not None else values
            b["syn"] = plan.add(f"path{path.index}.synapses", max(4, records.nbytes),
                                records.view(np.uint8) if records.nbytes else None)
    for path in plan.pathways:
        owner = path.state_owner
        if owner is not None:
            # the owner's record of each of this pathway's rows (both layouts list the same edges)
            path.syn_fields, path.syn_stride = owner.syn_fields, owner.syn_stride
            path.buffers["syn"] = owner.buffers["syn"]
            owner_row = np.empty(owner.edge_count, np.int64)
            owner_row[owner.order] = np.arange(owner.edge_count, dtype=np.int64)
            rec = owner_row[path.order].astype(np.uint32)
            path.buffers["rec_row"] = plan.add(f"path{path.index}.record_row", max(4, rec.nbytes),
                                               rec if rec.size else None)
    # slot tables of counting groups: per (source, delay group, target block) segment, the
    # count and up to SLOT_TARGETS block-local targets (or a longer segment's first row) in 32
    # bytes, one contiguous region per XCD (filled on the device once the topology exists)
    plan.queues.clear()
    for group in delivery_groups(plan):
        limits = queue_limits(plan, group)
        if limits is not None:
            # queued events: per arrival slot and target block a counter and up to `cap`
            # 8-byte records (the exact bound `limit` once an overflow has enlarged it)
            tpop = plan.populations[group[0].target]
            depth = push_depth(group)
            exact = (depth + 1) * tpop.blocks * limits[1] * 8
            cap = limits[1] if exact <= QUEUE_BUDGET_BYTES else min(limits[1], QUEUE_CAPACITY)
            info = dict(limit=limits[1], cap=cap, depth=depth)
            plan.queues[group[0].index] = info
            group[0].buffers["queue_count"] = plan.add(f"path{group[0].index}.queue_count", depth * tpop.blocks * 4)
            group[0].buffers["queue"] = plan.add(f"path{group[0].index}.queue_records",
                                                 max(8, depth * tpop.blocks * info["cap"] * 8))
            # a block's records sorted by target when they exceed one staging window
            group[0].buffers["queue_scratch"] = plan.add(f"path{group[0].index}.queue_scratch",
                                                         max(8, tpop.blocks * info["cap"] * 8))
            continue
        if not counting_group(group):
            if _edge_loop_candidate(plan):
                # row slots for the edge-keyed lists of the split loop
                for path in group:
                    path.row_slots = True
                    path.slot_entries = XCDS * path.scount * len(path.dvals) * per_xcd(plan)
                    path.buffers["slot"] = plan.add(f"path{path.index}.slots", path.slot_entries * 32)
            continue
        if push_group(plan, group):
            # pushed counts: per arrival slot, target block and pathway, one u32 per target
            tpop = plan.populations[group[0].target]
            arrivals = push_depth(group) * tpop.blocks * len(group) * plan.shape.block * 4
            group[0].buffers["arrivals"] = plan.add(f"path{group[0].index}.arrivals", arrivals)
            continue
        for path in group:
            path.slot_entries = XCDS * path.scount * len(path.dvals) * per_xcd(plan)
            path.buffers["slot"] = plan.add(f"path{path.index}.slots", path.slot_entries * 32)
    for k, code in enumerate(plan.synapse_codes):
        if code.kind == "summed":
            offsets, rows = endpoint_layout(code.path, code.to_pre)
            code.buffers["off"] = plan.add(f"summed{k}.offsets", offsets.nbytes, offsets)
            code.buffers["rows"] = plan.add(f"summed{k}.rows", max(4, rows.nbytes), rows if rows.size else None)
    for post in plan.post_paths:
        offsets, rows = post_layout(post.pre) if post.delays is None else post_group_layout(post)
        post.buffers["off"] = plan.add(f"post{post.index}.offsets", offsets.nbytes, offsets)
        post.buffers["rows"] = plan.add(f"post{post.index}.rows", max(4, rows.nbytes), rows if rows.size else None)
        if post.pending is not None:
            offsets, ids, post.pending_ticks = post_pending_layout(plan, post)
            post.buffers["pend_off"] = plan.add(f"post{post.index}.pending_offsets", offsets.nbytes, offsets)
            post.buffers["pend"] = plan.add(f"post{post.index}.pending", max(4, ids.nbytes), ids if ids.size else None)
    for group in delivery_groups(plan):
        group[0].pending_ticks = 0
        group[0].pending_sources = False
        sources = pending_source_layout(plan, group) if any(path.pending is not None for path in group) \
            and pending_as_sources(plan, group) else None
        if sources is not None:
            # pending sources per tick, looked up through the segment (or slot) tables like fired ones
            offsets, ids, group[0].pending_ticks = sources
            group[0].pending_sources = True
            group[0].buffers["pend_off"] = plan.add(f"path{group[0].index}.pending_offsets", offsets.nbytes, offsets)
            group[0].buffers["pend"] = plan.add(f"path{group[0].index}.pending", max(4, ids.nbytes),
                                                ids if ids.size else None)
        elif any(path.pending is not None for path in group):
            require(all(path.topology[0] == "explicit" for path in group if path.pending is not None),
                    "pending events of ordered or multi-delay groups need an explicit topology")
            offsets, entries, group[0].pending_ticks = pending_layout(plan, group)
            group[0].buffers["pend_off"] = plan.add(f"path{group[0].index}.pending_offsets", offsets.nbytes, offsets)
            group[0].buffers["pend"] = plan.add(f"path{group[0].index}.pending", max(8, entries.nbytes),
                                                entries if entries.size else None)


def syn_record_dtype(path: PathwayPlan) -> np.dtype:
    """NumPy view of a pathway's synapse-state records (row order)."""
    names = list(path.syn_fields)
    return np.dtype({"names": names, "formats": [NUMPY[path.syn_fields[n][1]] for n in names],
                     "offsets": [path.syn_fields[n][0] for n in names], "itemsize": path.syn_stride})


def syn_ref(path: PathwayPlan, name: str, const: bool = False) -> str:
    """C pointer to synapse state `name` of row `row`."""
    offset, dtype = path.syn_fields[name]
    return (f"atlas::field<{'const ' if const else ''}{CTYPE[dtype]}>(tab, {path.buffers['syn']}, "
            f"{record_index(path)}, {path.syn_stride}u, {offset}u)")


def record_index(path: PathwayPlan) -> str:
    """C expression of the synapse-state record of `row`: the row itself, or through the row map
    of a pathway whose states live in another pathway's rows."""
    if path.state_owner is None:
        return "row"
    return f"atlas::buf<const u32>(tab, {path.buffers['rec_row']})[row]"


def post_layout(pre: PathwayPlan) -> tuple[np.ndarray, np.ndarray]:
    """Incoming edges of every target of the synapse (local target index), edges ascending
    (edge_csr, executor.rs:6168-6183), as row positions of the pre pathway's layout.
    Returns (offsets u32[tcount + 1], rows u32[E])."""
    if pre.post_major:
        # an on_post event writes only its own edge's synapse states, so the edges of a target
        # may run in any order: here their rows ascending, one contiguous run per target
        tgt = np.asarray(pre.topology[2], np.int64)
        offsets = np.zeros(pre.tcount + 1, np.int64)
        np.cumsum(np.bincount(tgt, minlength=pre.tcount), out=offsets[1:])
        return offsets.astype(np.uint32), np.arange(pre.edge_count, dtype=np.uint32)
    return endpoint_layout(pre, to_pre=False)


def post_group_layout(post: PostPlan) -> tuple[np.ndarray, np.ndarray]:
    """The incoming edges of every target per delay group of an on_post pathway with per-edge
    delays, as row positions: offsets u32[groups * (tcount + 1)] (group g's table at g * (tcount + 1),
    positions into one rows array) and rows u32[E], ascending within each (group, target).  The
    events of one tick touch distinct edges, so their order does not matter."""
    pre = post.pre
    tgt = np.asarray(pre.topology[2], np.int64)
    lut = {value: g for g, value in enumerate(post.dvals)}
    group = np.array([lut[int(v)] for v in np.asarray(post.delays, np.int64)], np.int64)
    row_of_edge = np.empty(pre.edge_count, np.int64)
    row_of_edge[pre.order] = np.arange(pre.edge_count, dtype=np.int64)
    key = group * pre.tcount + tgt
    by_key = np.lexsort((row_of_edge, key))
    counts = np.bincount(key, minlength=len(post.dvals) * pre.tcount).reshape(len(post.dvals), pre.tcount)
    offsets = np.zeros((len(post.dvals), pre.tcount + 1), np.int64)
    offsets[:, 1:] = np.cumsum(counts, axis=1)
    offsets += np.concatenate([[0], np.cumsum(counts.sum(axis=1))[:-1]])[:, None]
    return offsets.reshape(-1).astype(np.uint32), row_of_edge[by_key].astype(np.uint32)


def endpoint_layout(pre: PathwayPlan, to_pre: bool) -> tuple[np.ndarray, np.ndarray]:
    """The edges of every target (or, with ``to_pre``, every source) of the synapse, local
    index, edges ascending, as row positions of the pre pathway's layout: (offsets
    u32[endpoints + 1], rows u32[E])."""
    _, src, tgt = pre.topology
    ends = src if to_pre else tgt
    count = pre.scount if to_pre else pre.tcount
    row_of_edge = np.empty(pre.edge_count, np.int64)
    row_of_edge[pre.order] = np.arange(pre.edge_count, dtype=np.int64)
    by_end = np.argsort(ends, kind="stable")   # edges ascending within an endpoint
    offsets = np.zeros(count + 1, np.int64)
    np.cumsum(np.bincount(ends, minlength=count), out=offsets[1:])
    return offsets.astype(np.uint32), row_of_edge[by_end].astype(np.uint32)


def _var_dtype(pop: PopulationPlan, name: str) -> str:
    for sname, dtype, _ in pop.states:
        if sname == name:
            return dtype
    if name in pop.scalar_params:
        return pop.scalar_params[name][0]
    return pop.vector_params[name][0]


def _population_inputs(pop: PopulationPlan, state_expr) -> dict:
    inputs = {"dt": (hexlit(pop.dt), "f64"), "t": ("t", "f64"), "N": (hexlit(float(pop.count)), "index"),
              "i": ("(double)i", "index")}
    for name, dtype, _ in pop.states:
        inputs[name] = (state_expr(name, dtype), dtype)
    for name, (dtype, value) in pop.scalar_params.items():
        inputs[name] = (hexlit(value), dtype)
    for name, (dtype, _) in pop.vector_params.items():
        inputs[name] = (f"atlas::buf<const double>(tab, {pop.buffers['param:' + name]})[i]", dtype)
    if pop.refractory is not None:
        inputs["lastspike"] = (f"atlas::buf<const double>(tab, {pop.buffers['lastspike']})[i]", "f64")
        inputs["not_refractory"] = ("(nr ? 1.0 : 0.0)", "bool")
    return inputs


# operations a scalar statement evaluated on the device may use: those whose results the host's
# and the device's f64 arithmetic give alike (no transcendental, whose host libm may differ by an ulp)
_DEVICE_SCALAR_OPS = frozenset({"literal", "boolean", "integer", "load", "rand", "add", "sub", "mul", "div", "neg",
                                "abs", "not", "gt", "ge", "lt", "le", "eq", "ne", "and", "or", "f32_to_f64",
                                "f64_to_f32", "bool_to_f64", "index_to_f64", "tick_to_f64", "clip", "sqrt", "floor",
                                "ceil", "mod", "floordiv"})


def _expr_ops(expr, ops: set, loads: set) -> None:
    if isinstance(expr, dict):
        if "op" in expr:
            ops.add(expr["op"])
            if expr["op"] == "load":
                loads.add(expr["name"])
        for v in expr.values():
            _expr_ops(v, ops, loads)
    elif isinstance(expr, list):
        for v in expr:
            _expr_ops(v, ops, loads)


def _scalar_env(pop: PopulationPlan, code: dict) -> dict:
    """Host values of a program's scalar statements (Program::prepare, executor.rs:5488-5515).  A
    statement drawing random numbers, or reading one that does, changes every tick: it is kept for
    the device (under the key "\0device"), where the program evaluates it with the draw index 0."""
    env = {"dt": pop.dt, "N": float(pop.count)}
    for name, (dtype, value) in pop.scalar_params.items():
        env[name] = value
    device, names = [], set()
    for statement in code["scalar"]:
        ops, loads = set(), set()
        _expr_ops(statement["value"], ops, loads)
        if "rand" in ops or loads & names or ops & _RANDOM_OPS:
            require(ops <= _DEVICE_SCALAR_OPS, "random draws in scalar statements are supported with rand() and "
                    "arithmetic only")
            device.append(statement)
            names.add(statement["target"])
            continue
        value = eval_scalar(statement["value"], env)
        if statement["dtype"] == "f32":
            value = struct.unpack("<f", struct.pack("<f", value))[0]
        env[statement["target"]] = value
    if device:
        env["\0device"] = device
    return env


def _with_scalars(inputs: dict, env: dict, code: dict) -> dict:
    out = dict(inputs)
    for statement in code["scalar"]:
        if statement["target"] in env:
            out[statement["target"]] = (hexlit(env[statement["target"]]), statement["dtype"])
    return out


def _population_code(plan: Plan, pop: PopulationPlan) -> str:
    b = pop.buffers
    L: list[str] = []
    L.append(f"struct Pop{pop.index} {{")
    L.append(f"    static constexpr u32 N = {pop.count}u, NB = {pop.blocks}u, R = {pop.ring}u;")
    L.append(f"    static constexpr int CNT = {b['spk_cnt']}, IDS = {b['spk_ids']}, SMALL = {b['spk_small']}, "
             f"FAULT = {plan.fault_buffer};")
    L.append(f"    static constexpr int REC = {b.get('rec', -1)};")
    L.append(f"    static constexpr u32 REC_WORDS = {b['rec_words']}u;")
    L.append(f"    static constexpr i64 WIN0 = {pop.window_start}LL;")
    # ---- state monitor
    L.append("    __device__ static void record(const u64* __restrict__ tab, i64 tick, u32 base, u32 n) {")
    if "mon_entries" in b:
        L.append(f"        if (tick < WIN0) return;")
        L.append(f"        const u32 blk = base / ATLAS_BLOCK;")
        L.append(f"        const u32* off = atlas::buf<const u32>(tab, {b['mon_offsets']});")
        L.append(f"        const u32* ent = atlas::buf<const u32>(tab, {b['mon_entries']});")
        L.append(f"        const u64 row = (u64)(tick - WIN0) * {len(pop.monitor_record)}u;")
        L.append("        for (u32 e = off[blk] + threadIdx.x; e < off[blk + 1]; e += ATLAS_WG) {")
        L.append("            const u32 r = ent[2 * e], i = ent[2 * e + 1];")
        for name in pop.monitor_vars:
            dtype = _var_dtype(pop, name)
            ct = CTYPE[dtype]
            if f"state:{name}" in b:
                src = f"atlas::buf<const {ct}>(tab, {b['state:' + name]})[i]"
            elif name in pop.scalar_params:
                src = f"({ct})({hexlit(pop.scalar_params[name][1])})"
            else:
                src = f"({ct})atlas::buf<const double>(tab, {b['param:' + name]})[i]"
            L.append(f"            atlas::buf<{ct}>(tab, {b['sample:' + name]})[row + r] = {src};")
        L.append("        }")
    else:
        L.append("        (void)tab; (void)tick; (void)base; (void)n;")
    L.append("    }")
    # ---- State / load / step / store (update + threshold [+ fused reset])
    L.append(f"    static constexpr bool RESET_FUSED = {'true' if pop.reset_fused else 'false'};")
    L.append("    struct State {")
    for name, dtype, _ in pop.states:
        L.append(f"        {CTYPE[dtype]} st_{name};")
    if pop.refractory is not None:
        L.append("        int until;")
    if pop.generator is not None:
        L.append("        u32 cursor, end, next;   // spike generator: this neuron's next scheduled spike")
    L.append("    };")
    L.append("    __device__ static void load(const u64* __restrict__ tab, u32 i, State& st) {")
    for name, dtype, _ in pop.states:
        L.append(f"        st.st_{name} = atlas::buf<const {CTYPE[dtype]}>(tab, {b['state:' + name]})[i];")
    if pop.refractory is not None:
        L.append(f"        st.until = atlas::buf<const int>(tab, {b['until']})[i];")
    if pop.generator is not None:
        L.append(f"        st.cursor = atlas::buf<const u32>(tab, {b['gen_cursor']})[i];")
        L.append(f"        st.end = atlas::buf<const u32>(tab, {b['gen_offsets']})[i + 1];")
        L.append(f"        st.next = st.cursor < st.end ? atlas::buf<const u32>(tab, {b['gen_ticks']})[st.cursor] "
                 f": 0xFFFFFFFFu;")
    L.append("    }")
    # the deadline of a spike at this tick, read once per tick from the run's table when it has one
    if "until_table" in b:
        L.append("    __device__ static int until_next(const u64* __restrict__ tab, i64 tick) {")
        L.append(f"        return atlas::uniform_load<int>(atlas::buf<const int>(tab, {b['until_table']}) + "
                 f"(tick - {pop.start_tick}LL));")
        L.append("    }")
    else:
        L.append("    __device__ static int until_next(const u64* __restrict__ tab, i64 tick) "
                 "{ (void)tab; (void)tick; return 0; }")
    L.append("    __device__ static bool step(const u64* __restrict__ tab, u32 i, double t, i64 tick, State& st, "
             "u32& fault, int until_next) {")
    L.append("        (void)tick; (void)fault; (void)t; (void)until_next;")
    if pop.refractory is not None:
        L.append("        bool nr = tick >= (i64)st.until;")
    state_in = lambda n, dt: f"(double)st.st_{n}"  # noqa: E731
    written = set()

    def regular_in_step(place: str, prefix: str) -> None:
        # run_regularly code at this place, on the states in registers (run_program_neurons)
        for k, (code, where) in enumerate(pop.regular):
            if where != place:
                continue
            env = _scalar_env(pop, code)
            inputs = _with_scalars(_population_inputs(pop, state_in), env, code)
            prog = DeviceProgram(inputs, L, f"{prefix}{k}_", rng=(plan.rng_seed, "i"))
            prog.scalar_statements(env)
            prog.statements(code["vector"])
            for name in code["effects"]["writes"]:
                dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
                L.append(f"        st.st_{name} = {commit_expr(dtype, prog.symbols[name][0])};")
                written.add(name)

    regular_in_step("pre", "ra")
    if pop.update is not None:
        env = _scalar_env(pop, pop.update)
        inputs = _with_scalars(_population_inputs(pop, state_in), env, pop.update)
        prog = DeviceProgram(inputs, L, "u", rng=(plan.rng_seed, "i"))
        prog.scalar_statements(env)
        prog.statements(pop.update["vector"])
        for name in pop.update["effects"]["writes"]:
            require(name in {s_[0] for s_ in pop.states}, f"update writes {name!r}")
            dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
            L.append(f"        st.st_{name} = {commit_expr(dtype, prog.symbols[name][0])};")
            written.add(name)
    regular_in_step("mid", "rb")

    def monitor_record(k: int, variables: list, value_of, indent: str) -> None:
        # EventMonitor k: one record (tick, neuron, the monitored values as f64) appended
        width = 1 + len(variables)
        L.append(f"{indent}{{ const u32 at = __hip_atomic_fetch_add(atlas::buf<u32>(tab, {b[f'emon_count:{k}']}), 1u, "
                 "__ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);")
        L.append(f"{indent}  if (at < {pop.event_monitor_capacity(k)}u) {{")
        L.append(f"{indent}    const atlas::gptr<double> r = atlas::buf<double>(tab, {b[f'emon:{k}']}) + (u64)at * {width}u;")
        L.append(f"{indent}    r[0] = __longlong_as_double((long long)((u64)(u32)tick << 32 | i));")
        for v, name in enumerate(variables):
            L.append(f"{indent}    r[{v + 1}] = {value_of(name)};")
        L.append(f"{indent}  }}")
        L.append(f"{indent}}}")

    def register_value(name: str) -> str:
        if name in {s_[0] for s_ in pop.states}:
            return f"(double)st.st_{name}"
        if name in pop.scalar_params:
            return hexlit(pop.scalar_params[name][1])
        return f"atlas::buf<const double>(tab, {b['param:' + name]})[i]"

    # custom events: each condition on the updated states (before any reset), its flag for the
    # resets slot, and the EventMonitors recording it at the threshold
    for k, (event, threshold_code, _) in enumerate(pop.custom_events):
        prog = DeviceProgram(_population_inputs(pop, state_in), L, f"ce{k}_", rng=(plan.rng_seed, "i"))
        prog.statements(threshold_code["vector"])
        L.append(f"        const bool event{k} = {prog.symbols['_cond'][0]} != 0.0;")
        L.append(f"        atlas::buf<byte_t>(tab, {b[f'evt:{k}']})[i] = event{k} ? (byte_t)1 : (byte_t)0;")
        mons = [(m, variables) for m, (_, variables, ev, when) in enumerate(pop.event_monitors)
                if ev == event and when == "thresholds"]
        if mons:
            L.append(f"        if (event{k}) {{")
            for m, variables in mons:
                monitor_record(m, variables, register_value, "            ")
            L.append("        }")
    fired = "false"
    if pop.generator is not None:
        # the neuron fires when its next scheduled tick is this one (ticks lie inside the run)
        L.append("        const bool fired = st.next == (u32)tick;")
        L.append("        if (fired) ++st.cursor;")
        fired = "fired"
    if pop.threshold is not None:
        prog = DeviceProgram(_population_inputs(pop, state_in), L, "h", rng=(plan.rng_seed, "i"))
        prog.statements(pop.threshold["vector"])
        cond = prog.symbols["_cond"][0]
        gate = " && nr" if pop.refractory is not None else ""
        L.append(f"        const bool fired = ({cond} != 0.0){gate};")
        fired = "fired"
        L.append("        if (fired) {")
        for k, (_, variables, event, when) in enumerate(pop.event_monitors):
            # EventMonitor: the neuron's monitored values at the threshold, before the reset
            if event == "spike" and when == "thresholds":
                monitor_record(k, variables, register_value, "            ")
        if pop.refractory is not None:
            period = pop.refractory[0]
            L.append(f"            __builtin_nontemporal_store(t, atlas::buf<double>(tab, {b['lastspike']}) + i);")
            if "until_table" in b:
                L.append("            st.until = until_next;")
            else:
                L.append(f"            st.until = (int)atlas::refractory_until(tick, t, {hexlit(pop.dt)}, "
                         f"{hexlit(pop.dt)}, {period}ull, fault);")
            L.append(f"            __builtin_nontemporal_store(st.until, atlas::buf<int>(tab, {b['until']}) + i);")
            L.append("            nr = false;")
        if pop.reset is not None and pop.reset_fused:
            env = _scalar_env(pop, pop.reset)
            inputs = _with_scalars(_population_inputs(pop, state_in), env, pop.reset)
            prog = DeviceProgram(inputs, L, "z", indent="            ", rng=(plan.rng_seed, "i"))
            prog.scalar_statements(env)
            prog.statements(pop.reset["vector"])
            for name in pop.reset["effects"]["writes"]:
                require(name in {s_[0] for s_ in pop.states}, f"reset writes {name!r}")
                dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
                L.append(f"            st.st_{name} = {commit_expr(dtype, prog.symbols[name][0])};")
                written.add(name)
        L.append("        }")
    L.append(f"        return {fired};")
    L.append("    }")
    L.append("    __device__ static void store(const u64* __restrict__ tab, u32 i, u32 j, const State& st, "
             "byte_t* post) {")
    L.append("        (void)tab; (void)i; (void)j; (void)st; (void)post;")
    for name in sorted(written | set(pop.lds_states) | pop.fused_writes):
        dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
        if name in pop.lds_states:
            L.append(f"        reinterpret_cast<{CTYPE[dtype]}*>(post + {pop.lds_states[name]})[j] = st.st_{name};")
        else:
            # streamed once per tick: a non-temporal store leaves no dirty L2 line for the
            # end-of-kernel writeback (measured: 16.2 -> 15.5 us per config-3 tick)
            L.append(f"        __builtin_nontemporal_store(st.st_{name}, "
                     f"atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]}) + i);")
    if pop.generator is not None:
        L.append(f"        atlas::buf<u32>(tab, {b['gen_cursor']})[i] = st.cursor;")
    L.append("    }")
    # the split persistent loop's end: every state it may have changed straight to memory (the
    # per-tick kernel stages the states an ordered group writes in LDS instead)
    L.append("    __device__ static void store_mem(const u64* __restrict__ tab, u32 i, const State& st) {")
    L.append("        (void)tab; (void)i; (void)st;")
    for name in sorted(written | set(pop.lds_states) | pop.fused_writes):
        dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
        L.append(f"        __builtin_nontemporal_store(st.st_{name}, atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]}) + i);")
    if pop.generator is not None:
        L.append(f"        atlas::buf<u32>(tab, {b['gen_cursor']})[i] = st.cursor;")
    L.append("    }")
    # several clocks: a step that delivers into the block without updating it stages these
    # states in LDS unchanged
    L.append("    __device__ static void stage(const u64* __restrict__ tab, u32 i, u32 j, byte_t* post) {")
    L.append("        (void)tab; (void)i; (void)j; (void)post;")
    for name, offset in pop.lds_states.items():
        dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
        L.append(f"        reinterpret_cast<{CTYPE[dtype]}*>(post + {offset})[j] = "
                 f"atlas::buf<const {CTYPE[dtype]}>(tab, {b['state:' + name]})[i];")
    L.append("    }")
    L.append("    __device__ static void writeback(const u64* __restrict__ tab, u32 i, u32 j, const byte_t* post) {")
    L.append("        (void)tab; (void)i; (void)j; (void)post;")
    for name, offset in pop.lds_states.items():
        dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
        L.append(f"        __builtin_nontemporal_store(reinterpret_cast<const {CTYPE[dtype]}*>(post + {offset})[j], "
                 f"atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]}) + i);")
    L.append("    }")
    # ---- reset
    # ---- PoissonInput programs (executor.rs:4121-4137, run_program_neurons over every neuron)
    L.append("    __device__ static void poisson(const u64* __restrict__ tab, u32 i, double t, i64 tick, u32& fault) {")
    L.append("        (void)tab; (void)i; (void)tick; (void)t; (void)fault;")
    for k, code in enumerate(pop.poisson_inputs):
        L.append("        {")
        for name, dtype, _ in pop.states:
            L.append(f"            {CTYPE[dtype]} st_{name} = atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]})[i];")
        if pop.refractory is not None:
            L.append(f"            const bool nr = tick >= (i64)atlas::buf<const int>(tab, {b['until']})[i];")
        env = _scalar_env(pop, code)
        inputs = _with_scalars(_population_inputs(pop, lambda n, dt: f"(double)st_{n}"), env, code)
        prog = DeviceProgram(inputs, L, f"q{k}_", indent="            ", rng=(plan.rng_seed, "i"))
        prog.scalar_statements(env)
        prog.statements(code["vector"])
        for name in code["effects"]["writes"]:
            dtype = next(s[1] for s in pop.states if s[0] == name)
            L.append(f"            atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]})[i] = "
                     f"{commit_expr(dtype, prog.symbols[name][0])};")
        L.append("        }")
    L.append("    }")
    # ---- run_regularly code at the end of the tick, on the states in memory
    L.append("    __device__ static void regular_end(const u64* __restrict__ tab, u32 i, double t, i64 tick, u32& fault) {")
    L.append("        (void)tab; (void)i; (void)tick; (void)t; (void)fault;")
    for k, (code, where) in enumerate(pop.regular):
        if where != "end":
            continue
        L.append("        {")
        for name, dtype, _ in pop.states:
            L.append(f"            {CTYPE[dtype]} st_{name} = atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]})[i];")
        if pop.refractory is not None:
            L.append(f"            const bool nr = tick >= (i64)atlas::buf<const int>(tab, {b['until']})[i];")
        env = _scalar_env(pop, code)
        inputs = _with_scalars(_population_inputs(pop, lambda n, dt: f"(double)st_{n}"), env, code)
        prog = DeviceProgram(inputs, L, f"rc{k}_", indent="            ", rng=(plan.rng_seed, "i"))
        prog.scalar_statements(env)
        prog.statements(code["vector"])
        for name in code["effects"]["writes"]:
            dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
            L.append(f"            atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]})[i] = "
                     f"{commit_expr(dtype, prog.symbols[name][0])};")
        L.append("        }")
    L.append("    }")
    L.append("    __device__ static void reset(const u64* __restrict__ tab, u32 i, double t, i64 tick, u32& fault) {")
    L.append("        (void)tick; (void)t; (void)fault;")
    if pop.reset is not None:
        for name, dtype, _ in pop.states:
            L.append(f"        {CTYPE[dtype]} st_{name} = atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]})[i];")
        if pop.refractory is not None:
            L.append(f"        const bool nr = tick >= (i64)atlas::buf<const int>(tab, {b['until']})[i];")
        env = _scalar_env(pop, pop.reset)
        inputs = _with_scalars(_population_inputs(pop, lambda n, dt: f"(double)st_{n}"), env, pop.reset)
        prog = DeviceProgram(inputs, L, "z", rng=(plan.rng_seed, "i"))
        prog.scalar_statements(env)
        prog.statements(pop.reset["vector"])
        for name in pop.reset["effects"]["writes"]:
            require(name in {s[0] for s in pop.states}, f"reset writes {name!r}")
            dtype = next(s[1] for s in pop.states if s[0] == name)
            L.append(f"        atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]})[i] = "
                     f"{commit_expr(dtype, prog.symbols[name][0])};")
    L.append("    }")
    _custom_phase_code(plan, pop, L)
    _event_ring_code(pop, L)
    L.append("};")
    return "\n".join(L)


def _event_ring_code(pop: PopulationPlan, L: list) -> None:
    """Pop::publish_events, run at the end of the update for every block: the block's neurons
    whose custom event fired this tick (their flags, written by the same work-items), ascending,
    into that event's ring in the spike ring's layout (the slot's ids, the first 8 per block, the
    count), for the pathways the event triggers.  Published where the spikes are, so a pathway
    on a custom event reads its ring as a spike pathway reads the spike ring, delay 0 included."""
    b = pop.buffers
    L.append(f"    static constexpr bool EVENT_RINGS = {'true' if pop.event_rings else 'false'};")
    L.append("    __device__ static void publish_events(const u64* __restrict__ tab, i64 tick, u32 blk) {")
    L.append("        (void)tab; (void)tick; (void)blk;")
    if not pop.event_rings:
        L.append("    }")
        return
    L.append("        __shared__ u32 evc_[ATLAS_WAVES];")
    L.append("        const u32 base = blk * ATLAS_BLOCK;")
    L.append("        const u32 n = (N - base < ATLAS_BLOCK) ? N - base : ATLAS_BLOCK;")
    L.append("        const u32 lane = __lane_id(), wave = threadIdx.x >> 6;")
    for k, ring in sorted(pop.event_rings.items()):
        L.append("        {")
        L.append(f"            const u32 slot = (u32)(tick % {ring});")
        L.append(f"            u32* ids = atlas::buf<u32>(tab, {b[f'ering_ids:{k}']}) + (u64)slot * N + base;")
        L.append(f"            u32* small = atlas::buf<u32>(tab, {b[f'ering_small:{k}']}) + ((u64)slot * NB + blk) * 8u;")
        L.append("            u32 before = 0;")
        L.append("            for (u32 r = 0; r < ATLAS_ROUNDS; ++r) {")
        L.append("                const u32 j = r * ATLAS_WG + threadIdx.x;")
        L.append(f"                const bool f = j < n && atlas::buf<const byte_t>(tab, {b[f'evt:{k}']})[base + j] != 0;")
        L.append("                const u64 m = __ballot(f);")
        L.append("                atlas::lds_barrier();   // the previous round's counts are read")
        L.append("                if (lane == 0) evc_[wave] = (u32)__popcll(m);")
        L.append("                atlas::lds_barrier();")
        L.append("                u32 mine = before;")
        L.append("                for (u32 w = 0; w < ATLAS_WAVES; ++w) {")
        L.append("                    const u32 c = evc_[w];")
        L.append("                    if (w < wave) mine += c;")
        L.append("                    before += c;")
        L.append("                }")
        L.append("                if (f) {")
        L.append("                    const u32 at = mine + (u32)__popcll(m & ((1ull << lane) - 1ull));")
        L.append("                    ids[at] = base + j;")
        L.append("                    if (at < 8u) small[at] = base + j;")
        L.append("                }")
        L.append("            }")
        L.append(f"            if (threadIdx.x == 0) atlas::buf<u32>(tab, {b[f'ering_cnt:{k}']})[(u64)slot * NB + blk] = before;")
        L.append("            atlas::lds_barrier();   // every count read before the next event's")
        L.append("        }")
    L.append("    }")


def _custom_phase_code(plan: Plan, pop: PopulationPlan, L: list) -> None:
    """The resets slot of a population with custom events or end-of-tick EventMonitors
    (Pop::custom_phase, run by reset_phase for every block): the resets of the tick's events in
    schedule order (the spike reset on the tick's spikes unless fused, each custom event's
    run_on_event code on the neurons its flag marks; executor.rs:4157-4186), then the EventMonitors
    of the end slot on the states after them, then each custom event's stream bitmap row."""
    b = pop.buffers
    end_monitors = [(m, variables, event) for m, (_, variables, event, when) in enumerate(pop.event_monitors)
                    if when == "end"]
    custom = bool(pop.custom_events or end_monitors)
    L.append(f"    static constexpr bool CUSTOM = {'true' if custom else 'false'};")
    for k, (event, _, reset_code) in enumerate(pop.custom_events):
        if reset_code is None:
            continue
        L.append(f"    __device__ static void custom_reset{k}(const u64* __restrict__ tab, u32 i, double t, i64 tick, "
                 "u32& fault) {")
        L.append("        (void)tick; (void)t; (void)fault;")
        for name, dtype, _ in pop.states:
            L.append(f"        {CTYPE[dtype]} st_{name} = atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]})[i];")
        if pop.refractory is not None:
            L.append(f"        const bool nr = tick >= (i64)atlas::buf<const int>(tab, {b['until']})[i];")
        prog = DeviceProgram(_population_inputs(pop, lambda n, dt: f"(double)st_{n}"), L, f"cz{k}_",
                             rng=(plan.rng_seed, "i"))
        prog.statements(reset_code["vector"])
        for name in reset_code["effects"]["writes"]:
            dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
            L.append(f"        atlas::buf<{CTYPE[dtype]}>(tab, {b['state:' + name]})[i] = "
                     f"{commit_expr(dtype, prog.symbols[name][0])};")
        L.append("    }")
    L.append("    __device__ static void custom_phase(const u64* __restrict__ tab, i64 tick, double t, u32 blk) {")
    L.append("        (void)tab; (void)tick; (void)t; (void)blk;")
    if not custom:
        L.append("    }")
        return
    L.append("        u32 fault = 0;")
    L.append("        const u32 base = blk * ATLAS_BLOCK;")
    L.append("        const u32 n = (N - base < ATLAS_BLOCK) ? N - base : ATLAS_BLOCK;")
    if pop.has_spike_event:
        L.append("        const u32 slot = (u32)(tick % R);")
        L.append("        const u32 count = atlas::buf<u32>(tab, CNT)[(u64)slot * NB + blk];")
        L.append("        const u32* ids = atlas::buf<u32>(tab, IDS) + (u64)slot * N + base;")
    index = {event: k for k, (event, _, _) in enumerate(pop.custom_events)}
    for event in pop.reset_order:
        if event == "spike":
            if pop.reset is None or pop.reset_fused:
                continue
            L.append("        for (u32 k = threadIdx.x; k < count; k += ATLAS_WG) reset(tab, ids[k], t, tick, fault);")
        else:
            k = index[event]
            L.append("        for (u32 j = threadIdx.x; j < n; j += ATLAS_WG) {")
            L.append("            const u32 i = base + j;")
            L.append(f"            if (atlas::buf<const byte_t>(tab, {b[f'evt:{k}']})[i]) custom_reset{k}(tab, i, t, tick, fault);")
            L.append("        }")
        L.append("        __threadfence_block();")
        L.append("        __syncthreads();")

    def memory_value(name: str) -> str:
        if name in {s_[0] for s_ in pop.states}:
            dtype = next(s_[1] for s_ in pop.states if s_[0] == name)
            return f"(double)atlas::buf<const {CTYPE[dtype]}>(tab, {b['state:' + name]})[i]"
        if name in pop.scalar_params:
            return hexlit(pop.scalar_params[name][1])
        return f"atlas::buf<const double>(tab, {b['param:' + name]})[i]"

    for m, variables, event in end_monitors:
        width = 1 + len(variables)
        if event == "spike":
            L.append("        for (u32 k = threadIdx.x; k < count; k += ATLAS_WG) {")
            L.append("            const u32 i = ids[k];")
        else:
            L.append("        for (u32 j = threadIdx.x; j < n; j += ATLAS_WG) {")
            L.append("            const u32 i = base + j;")
            L.append(f"            if (!atlas::buf<const byte_t>(tab, {b[f'evt:{index[event]}']})[i]) continue;")
        L.append(f"            const u32 at = __hip_atomic_fetch_add(atlas::buf<u32>(tab, {b[f'emon_count:{m}']}), 1u, "
                 "__ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);")
        L.append(f"            if (at < {pop.event_monitor_capacity(m)}u) {{")
        L.append(f"                const atlas::gptr<double> r = atlas::buf<double>(tab, {b[f'emon:{m}']}) + (u64)at * {width}u;")
        L.append("                r[0] = __longlong_as_double((long long)((u64)(u32)tick << 32 | i));")
        for v, name in enumerate(variables):
            L.append(f"                r[{v + 1}] = {memory_value(name)};")
        L.append("            }")
        L.append("        }")
    if pop.custom_events:
        L.append("        if (tick >= WIN0) {")
        for k, _ in enumerate(pop.custom_events):
            L.append("            for (u32 w = threadIdx.x; w < (n + 31u) / 32u; w += ATLAS_WG) {")
            L.append("                u32 word = 0;")
            L.append("                for (u32 q = 0; q < 32u; ++q) {")
            L.append("                    const u32 j = w * 32u + q;")
            L.append(f"                    if (j < n && atlas::buf<const byte_t>(tab, {b[f'evt:{k}']})[base + j]) word |= 1u << q;")
            L.append("                }")
            L.append(f"                atlas::buf<u32>(tab, {b[f'evrec:{k}']})[(u64)(tick - WIN0) * REC_WORDS + base / 32u + w] = word;")
            L.append("            }")
        L.append("        }")
    L.append("        atlas::report(tab, FAULT, fault);")
    L.append("    }")


def _touched_post(path: PathwayPlan) -> tuple[set, set]:
    """Post-population states read and written by a pathway program."""
    reads = _reads(path.code)
    writes = set(path.code["effects"]["writes"])
    read_states = {path.post_aliases[a] for a in reads if a in path.post_aliases}
    write_states = {path.post_aliases[a] for a in writes if a in path.post_aliases}
    if "not_refractory_post" in reads:
        read_states.add("\0not_refractory")
    return read_states, write_states


def _reset_fusable(plan: Plan, pop: PopulationPlan) -> bool:
    """The reset may run right after the threshold (inside phase A) when no pathway into
    the population reads or writes a state the reset reads or writes: then the reset
    commutes with every delivery of the tick (AtlasIR.md section 5, effect algebra)."""
    if pop.reset is None:
        return False
    # custom events' run_on_event code may come before the spike reset in the resets slot
    if any(reset is not None for _, _, reset in pop.custom_events):
        return False
    reads = _reads(pop.reset)
    touched = ({n for n in reads if n in {s_[0] for s_ in pop.states}} |
               set(pop.reset["effects"]["writes"]))
    for path in plan.pathways:
        if path.target == pop.index:
            r, w = _touched_post(path)
            if touched & (r | w):
                return False
    for code in pop.poisson_inputs:
        if touched & (_reads(code) | set(code["effects"]["writes"])):
            return False
    return True


def edge_group(plan: Plan, group: list[PathwayPlan]) -> bool:
    """An ordered group the split persistent loop can deliver through edge-keyed lists
    (atlas_tick.h persistent_run_split with Group::EDGE): one delay of at least one tick, every
    program reading post states, at most one per-edge parameter (no synapse states) and
    constants, and writing post states only, at most four pathways of fewer than 2^30 edges each
    (the event key is pathway << 30 | edge id), no pending events.  Its events are applied per
    target in key order, which is the canonical order within a tick."""
    if counting_group(group) or plan.split or plan.multi_clock or len(group) > 4:
        return False
    delays = {d for path in group for d in path.dvals}
    if len(delays) != 1 or min(delays) < 1:
        return False
    for path in group:
        if path.syn_states or path.pending is not None or path.edge_count >= 1 << EDGE_KEY_BITS:
            return False
        if not set(path.code["effects"]["writes"]) <= set(path.post_aliases):
            return False
        if "\0not_refractory" in _touched_post(path)[0] or len(_edge_values(path)) > 1:
            return False
    return True


def _edge_slots(plan: Plan, group: list[PathwayPlan]) -> bool:
    """An edge group whose row slots are complete (built, no segment above SLOT_MAX_COUNT)."""
    return (all(path.row_slots and "slot" in path.buffers and path.index not in plan.slot_fallback for path in group)
            and edge_group(plan, group))


def _edge_loop_candidate(plan: Plan) -> bool:
    """Whether the plan may run the split loop with edge-keyed lists (checked again in full by
    persistent_eligible once the code is generated): one population, one ordered group into it
    that edge_group accepts, no on_post pathways or synapse codes."""
    if not PERSISTENT_EDGES or len(plan.populations) != 1 or plan.post_paths or plan.synapse_codes:
        return False
    groups = delivery_groups(plan)
    return (len(groups) == 1 and edge_group(plan, groups[0])
            and PERSISTENT_MIN_BLOCKS <= plan.total_blocks)


SLOT_TARGETS = 15   # targets held inline by one 32-byte slot (word 0 is the count)
SLOT_MAX_COUNT = 0xFFFF   # longer segments keep their first row in the slot, up to this count


def per_xcd(plan: "Plan") -> int:
    """Consecutive workgroup indices (blocks) per XCD: workgroup w runs on XCD w // per_xcd."""
    return (plan.total_blocks + XCDS - 1) // XCDS


def persistent_eligible(plan: Plan, groups: list, counting: list, split_loop: bool = False) -> bool:
    """Whether one cooperative launch may run many ticks with the block's states in registers
    (atlas_tick.h persistent_run).  The only memory a workgroup then reads from another inside a
    launch must be the spike ring (stamped words, so at most 2^20 neurons): one population whose deliveries are one counting group of
    one delay read through complete slot tables (one slot per fired source, or per fired source and pathway where the pathways'
    source ranges overlap), applied in registers (after the update
    for a delay >= 1, after the tick's own exchange for delay 0), the reset fused into the update, and nothing that reads or writes the
    states in memory during a tick (state monitors, event monitors, PoissonInputs, spike
    generators, on_post pathways, pending events, synapse codes run before each tick).  An ordered
    group runs only in the split loop, through edge-keyed lists (edge_group).  At least
    PERSISTENT_MIN_BLOCKS blocks
    (smaller networks are launch-latency bound either way) and at most RESIDENT_BLOCKS (every
    workgroup resident)."""
    if (plan.multi_clock or len(plan.populations) != 1 or plan.post_paths or len(groups) != 1
            or plan.synapse_codes):
        return False
    pop = plan.populations[0]
    # counted events applied in registers: after the update (delay >= 1), or, with delay 0, after
    # the tick's own exchange (the same Fused programs)
    edges = pop.fused_edges and split_loop
    if not (pop.fused_split if plan.split else (pop.fused_counts or edges)) or not (pop.reset is None or pop.reset_fused):
        return False
    if pop.poisson_inputs or pop.generator is not None or pop.event_monitors or pop.custom_events:
        return False
    if any(where == "end" for _, where in pop.regular):   # run on the states in memory after the reset
        return False
    if pop.monitor_record and pop.monitor_vars:
        return False
    if not PERSISTENT_MIN_BLOCKS <= plan.total_blocks <= RESIDENT_BLOCKS * 512 // plan.shape.wg:
        return False
    if pop.count > 1 << 20:   # stamped ring words carry 20-bit neuron indices
        return False
    for k, group in enumerate(groups):
        delays = {d for path in group for d in path.dvals}
        if not (counting[k] or edges) or len(delays) != 1 or (min(delays) < 1) != plan.split or group[0].pending_ticks:
            return False
        if not all("slot" in path.buffers and path.index not in plan.slot_fallback for path in group):
            return False
        if any(path.pending is not None for path in group):
            return False
    return True


def counting_group(group: list[PathwayPlan]) -> bool:
    """A group's events may be counted instead of ordered when every program reads
    no per-edge data (synapse states, non-constant per-edge parameters, random draws,
    which the counter RNG indexes by edge) and writes only post-synaptic states: each
    event into a target then applies the same function of the target's states, so the
    canonical order and any other order give bit-identical results."""
    for path in group:
        per_edge = {name for name, _, _ in path.syn_states} | set(path.edge_params)
        if _reads(path.code) & per_edge or draws_random(path.code["vector"]):
            return False
        if not set(path.code["effects"]["writes"]) <= set(path.post_aliases):
            return False
    return True


def push_group(plan: Plan, group: list[PathwayPlan]) -> bool:
    """Counting groups whose events come with several delays are delivered by push (the
    firing source's workgroup adds its out-edges to per-target counters of the arrival
    tick) rather than by pull, which would look up every (fired source, delay group)
    segment in every target block.  Needs every delay >= 1 tick and one kernel per tick,
    so a count pushed at tick t is only taken by a later launch."""
    delays = {d for path in group for d in path.dvals}
    return counting_group(group) and len(delays) > 1 and min(delays) >= 1 and not plan.split


QUEUE_CAPACITY = 8192   # initial records per (arrival slot, target block) of a queued group
# device bytes a queued group's records may take at their exact bound (in-edges per block for
# every arrival slot, plus the sort scratch): within it the queues never overflow and a run is
# never replayed; beyond it they start at QUEUE_CAPACITY and grow on overflow
QUEUE_BUDGET_BYTES = 32 << 30


def queue_limits(plan: Plan, group: list[PathwayPlan]) -> tuple[int, int] | None:
    """For an ordered group whose events come with several delays (all >= 1 tick, one kernel
    per tick): (the most events one target can receive in a tick, the most one target block
    can), i.e. in-edges per target and per block, since an edge carries at most one event
    per arrival tick.  None when the group is not queued: it is a counting group, it has one
    delay, or a target could receive more events than one LDS staging window holds."""
    delays = {d for path in group for d in path.dvals}
    if counting_group(group) or len(delays) < 2 or min(delays) < 1 or plan.split:
        return None
    if max(delays) >= 1 << 16 or plan.shape.block > 4096 or len(group) > 16:
        return None
    tpop = plan.populations[group[0].target]
    per_target = np.zeros(tpop.blocks * plan.shape.block, np.int64)
    for path in group:
        if path.topology[0] == "explicit":
            _, _, tgt = path.topology
            per_target[:tpop.count] += np.bincount(np.asarray(tgt, np.int64) + path.tstart,
                                                   minlength=tpop.count)[:tpop.count]
        else:
            per_target[path.tstart:path.tstart + path.tcount] += int(path.topology[1])
    if int(per_target.max(initial=0)) > 1 << plan.shape.cap_bits:
        return None
    per_block = per_target.reshape(tpop.blocks, plan.shape.block).sum(axis=1)
    return int(per_target.max(initial=0)), max(1, int(per_block.max(initial=0)))


def push_depth(group: list[PathwayPlan]) -> int:
    """Arrival-ring slots of a push group: the largest delay + 1."""
    return max(d for path in group for d in path.dvals) + 1


def delivery_groups(plan: Plan) -> list[list[PathwayPlan]]:
    """Adjacent (per target population, in schedule order) pathways that share their
    source population and touch disjoint post states are delivered together."""
    groups: list[list[PathwayPlan]] = []
    for pop in plan.populations:
        current: list[PathwayPlan] = []
        for path in [p for p in plan.pathways if p.target == pop.index]:
            ok = (bool(current) and current[0].source == path.source and current[0].event == path.event
                  and len(current) < 8)
            if ok and path.syn_states and any(other.synapse == path.synapse and other.syn_states for other in current):
                # pathways sharing synapse states run one after the other, as the reference does
                ok = False
            if ok:
                r2, w2 = _touched_post(path)
                for other in current:
                    r1, w1 = _touched_post(other)
                    if (w1 & (r2 | w2)) or (w2 & r1):
                        ok = False
            if ok:
                current.append(path)
            else:
                if current:
                    groups.append(current)
                current = [path]
        if current:
            groups.append(current)
    return groups


PREFETCH_LDS_LIMIT = 40 * 1024   # LDS bytes a group may use for its staged per-edge values


def _prefetch_layout(plan: Plan, group: list[PathwayPlan]) -> list | None:
    """Per pathway of an ordered group, the per-edge values (synapse states, per-edge
    parameters) its program reads, as (name, dtype, LDS byte offset) with one
    ATLAS_CAP-entry array each.  Every staged event belongs to one pathway, so the
    pathways' arrays overlap.  None when a value is not 4 or 8 bytes wide or the arrays
    would pass PREFETCH_LDS_LIMIT."""
    cap = 1 << plan.shape.cap_bits
    layout, size = [], 0
    for path in group:
        offset, mine = 0, []
        for name, dtype in sorted(_edge_values(path), key=lambda v: -np.dtype(NUMPY[v[1]]).itemsize):
            width = np.dtype(NUMPY[dtype]).itemsize
            if width not in (4, 8):
                return None
            mine.append((name, dtype, offset))
            offset += width * cap
        layout.append(mine)
        size = max(size, offset)
    if size == 0 or size > PREFETCH_LDS_LIMIT:
        return None
    return layout


def _prefetch_bytes(plan: Plan, group: list[PathwayPlan]) -> int:
    layout = _prefetch_layout(plan, group)
    if layout is None:
        return 0
    cap = 1 << plan.shape.cap_bits
    return max(sum(np.dtype(NUMPY[d]).itemsize * cap for _, d, _ in mine) for mine in layout)


def _edge_values(path: PathwayPlan) -> list:
    """The per-edge values (synapse states, per-edge parameters) a pathway's program reads,
    as (name, dtype)."""
    reads = _reads(path.code)
    values = [(name, dtype) for name, dtype, _ in path.syn_states if name in reads]
    values += [(name, "f64") for name in path.edge_params if name in reads]
    return values


def _word_expr(dtype: str, w: int, shift: int = 0) -> str:
    """A value of `dtype` held in the words v.w[w...] (at byte `shift` of word w), as double."""
    if dtype in ("f64", "i64"):
        bits = f"((u64)v.w[{w}] | (u64)v.w[{w + 1}] << 32)"
        return f"__longlong_as_double((long long){bits})" if dtype == "f64" else f"(double)(i64){bits}"
    return {"f32": f"(double)__uint_as_float(v.w[{w}])", "i32": f"(double)(int)v.w[{w}]",
            "bool": f"(double)((v.w[{w}] >> {8 * shift}) & 0xFFu)"}[dtype]


def _register_fetch(path: PathwayPlan, L: list, indent: str) -> tuple[int, dict, dict]:
    """Emit `fetch` lines loading the per-edge values of `row` the program reads into
    32-bit words v.w[...]: the row's synapse-state record whole (one cache line), then
    each per-edge parameter.  Returns (word count, name -> C expression of the value as
    double, name -> (dtype, first word))."""
    values = _edge_values(path)
    exprs, words = {}, {}
    w = 0
    if any(name in path.syn_fields for name, _ in values):
        n = path.syn_stride // 4
        base = f"atlas::field<const u32>(tab, {path.buffers['syn']}, {record_index(path)}, {path.syn_stride}u, 0u)"
        if n % 4 == 0:
            L.append(f"{indent}{{ const atlas::gptr<const uint4> r = (atlas::gptr<const uint4>){base};")
            for k in range(n // 4):
                L.append(f"{indent}  const uint4 x{k} = r[{k}]; v.w[{4 * k}] = x{k}.x; v.w[{4 * k + 1}] = x{k}.y; "
                         f"v.w[{4 * k + 2}] = x{k}.z; v.w[{4 * k + 3}] = x{k}.w;")
            L.append(f"{indent}}}")
        elif n % 2 == 0:
            L.append(f"{indent}{{ const atlas::gptr<const uint2> r = (atlas::gptr<const uint2>){base};")
            for k in range(n // 2):
                L.append(f"{indent}  const uint2 x{k} = r[{k}]; v.w[{2 * k}] = x{k}.x; v.w[{2 * k + 1}] = x{k}.y;")
            L.append(f"{indent}}}")
        else:
            L.append(f"{indent}v.w[0] = *{base};")
        for name, dtype in values:
            if name in path.syn_fields:
                offset = path.syn_fields[name][0]
                exprs[name] = _word_expr(dtype, offset // 4, offset % 4)
                words[name] = (dtype, offset // 4)
        w = n
    for name, dtype in values:
        if name in path.edge_params:
            L.append(f"{indent}{{ const u64 x = {_edge_param_bits(path, name)}; "
                     f"v.w[{w}] = (u32)x; v.w[{w + 1}] = (u32)(x >> 32); }}")
            exprs[name] = _word_expr("f64", w)
            words[name] = ("f64", w)
            w += 2
    return w, exprs, words


_RANDOM_OPS = frozenset({"rand", "randn", "binomial", "poisson"})


def draws_random(value) -> bool:
    """Whether an AtlasIR code object (or any part of one) draws from the counter RNG."""
    if isinstance(value, dict):
        return value.get("op") in _RANDOM_OPS or any(draws_random(v) for v in value.values())
    return isinstance(value, (list, tuple)) and any(draws_random(v) for v in value)


def _edge_rng(plan: Plan, path: PathwayPlan) -> tuple:
    """Counter-RNG binding of a synapse-domain program at `row`: the reference draws
    counter_uniform(seed, stream, tick, edge) for the iteration domains all_synapses and
    active_synapses (executor.rs:5071-5074, 5572-5577), with the edge index of the projection's
    own edge order.  Procedural rows are in that order (row_order_check); explicit layouts read
    it from the row's edge-id table.  None for a projection whose programs draw nothing."""
    if not path.random:
        return None
    if "edge_id" in path.buffers:
        return plan.rng_seed, f"atlas::buf<const u32>(tab, {path.buffers['edge_id']})[row]"
    require(path.order is None, "an explicit projection drawing random numbers needs its edge-id table")
    return plan.rng_seed, "row"


def _edge_param_expr(path: PathwayPlan, name: str) -> str:
    """C expression (double) of per-edge parameter `name` at `row`: a load, or the procedural
    uniform draw of a generated parameter."""
    if name in path.edge_gen:
        seed, stream, low, high = path.edge_gen[name]
        return f"atlas::edge_uniform({seed}ull, {stream}ull, (u64)row, {hexlit(low)}, {hexlit(high)})"
    return f"atlas::buf<const double>(tab, {path.buffers['eparam:' + name]})[row]"


def _edge_param_bits(path: PathwayPlan, name: str) -> str:
    """The same value's 64 bits (u64)."""
    if name in path.edge_gen:
        return f"(u64)__double_as_longlong({_edge_param_expr(path, name)})"
    return f"atlas::buf<const u64>(tab, {path.buffers['eparam:' + name]})[row]"


def _event_inputs(plan: Plan, path: PathwayPlan, staged: dict | None = None) -> dict:
    """Program inputs of one event (`row`, `neuron`, `post_*` registers).  `staged` maps
    per-edge values to C expressions that replace their loads from memory (values
    fetched ahead into LDS or registers)."""
    b = path.buffers
    src = plan.populations[path.source]
    tgt = plan.populations[path.target]
    inputs = {"dt": (hexlit(src.dt), "f64"), "t": ("t", "f64"), "N": (hexlit(float(path.edge_count)), "index"),
              "N_pre": (hexlit(float(path.scount)), "index"), "N_post": (hexlit(float(path.tcount)), "index"),
              "j": (f"(double)(neuron - {path.tstart}u)", "index")}
    for alias, state in path.post_aliases.items():
        dtype = next(s_[1] for s_ in tgt.states if s_[0] == state)
        inputs[alias] = (f"(double)post_{state}", dtype)
    for name, dtype, _ in path.syn_states:
        inputs[name] = (f"(double)*{syn_ref(path, name, const=True)}", dtype)
    for name, (dtype, _) in path.edge_params.items():
        inputs[name] = (_edge_param_expr(path, name), dtype)
    for name, expr in (staged or {}).items():
        inputs[name] = (expr, inputs[name][1])
    for name, (dtype, value) in path.scalar_params.items():
        inputs[name] = (hexlit(value), dtype)
    if tgt.refractory is not None:
        inputs["not_refractory_post"] = (
            f"(tick >= (i64)atlas::buf<const int>(tab, {tgt.buffers['until']})[neuron] ? 1.0 : 0.0)", "bool")
    return inputs


def _event_program(plan: Plan, path: PathwayPlan, L: list, indent: str, staged: dict | None = None) -> "DeviceProgram":
    """Emit the pathway's per-event program for one event (see _event_inputs)."""
    prog = DeviceProgram(_event_inputs(plan, path, staged), L, f"q{path.index}_", indent=indent,
                         rng=_edge_rng(plan, path))
    prog.statements(path.code["vector"])
    _event_commits(plan, path, prog, L, indent)
    return prog


def _event_commits(plan: Plan, path: PathwayPlan, prog: "DeviceProgram", L: list, indent: str) -> None:
    tgt = plan.populations[path.target]
    for name in path.code["effects"]["writes"]:
        value = prog.symbols[name][0]
        if name in path.post_aliases:
            state = path.post_aliases[name]
            dtype = next(s_[1] for s_ in tgt.states if s_[0] == state)
            L.append(f"{indent}post_{state} = {commit_expr(dtype, value)};")
        else:
            dtype = next(s_[1] for s_ in path.syn_states if s_[0] == name)
            L.append(f"{indent}*{syn_ref(path, name)} = {commit_expr(dtype, value)};")


SPLIT_EXPORTS = 3   # values an edge part may hand to the sequential part (ATLAS_CAP doubles of LDS each)


def _statement_reads(statement: dict) -> set:
    names = _reads({"scalar": [], "vector": [statement]})
    if statement.get("condition") is not None:
        names.add(statement["target"])   # a conditional assignment keeps the old value otherwise
    return names


def _split_plan(path: PathwayPlan) -> tuple[set, dict] | None:
    """Split an ordered pathway's program: the sequential statements are those that assign a
    post-synaptic state or read one (directly or through a symbol a sequential statement
    assigned); every other statement depends on the event's own edge only and can run for
    all staged events at once.  Returns (indices of the sequential statements, {index: the
    edge-local symbols that statement reads}) or None when more than SPLIT_EXPORTS values
    would cross over."""
    post = set(path.post_aliases) | {"not_refractory_post", "j"}
    dependent = set(post)
    sequential, needs = set(), {}
    for i, statement in enumerate(path.code["vector"]):
        reads = _statement_reads(statement)
        if reads & dependent or statement["target"] in post:
            sequential.add(i)
            needs[i] = sorted(reads - dependent)
            dependent.add(statement["target"])
        else:
            dependent.discard(statement["target"])
    if sum(len(v) for v in needs.values()) > SPLIT_EXPORTS:
        return None
    return sequential, needs


def _split_crossings(path: PathwayPlan) -> int:
    return sum(len(v) for v in _split_plan(path)[1].values())


def _split_code(plan: Plan, path: PathwayPlan, edge_exprs: dict, cap: int, L1: list, L2: list, indent: str) -> None:
    """Emit the edge part (L1: the statements of the event's own edge, from the fetched values
    `edge_exprs`, the stores of the synapse states they assign last, and the crossing values
    into LDS at the event's staging index `at`) and the sequential part (L2: the remaining
    statements, from the post-state registers and the crossing values; post-state and
    remaining synapse stores) of one pathway's program."""
    sequential, needs = _split_plan(path)
    statements = path.code["vector"]
    b = path.buffers
    tgt = plan.populations[path.target]
    local = {n for n, _ in _edge_values(path)}
    hidden = set(path.post_aliases) | {"not_refractory_post", "j"}
    inputs1 = {k: v for k, v in _event_inputs(plan, path, edge_exprs).items() if k not in hidden}
    prog1 = DeviceProgram(inputs1, L1, f"e{path.index}_", indent=indent, rng=_edge_rng(plan, path))
    crossing = []
    for i, statement in enumerate(statements):
        if i in sequential:
            for name in needs[i]:
                var, dtype = prog1.resolve(name)
                L1.append(f"{indent}reinterpret_cast<double*>(syn + {len(crossing) * 8 * cap})[at] = {var};")
                crossing.append((i, name, len(crossing), dtype))
        else:
            prog1.statements([statement])
    last = {statement["target"]: i for i, statement in enumerate(statements)}
    for name in path.code["effects"]["writes"]:
        if name in path.post_aliases or last.get(name) in sequential:
            continue
        var = prog1.resolve(name)[0]
        dtype = next(s_[1] for s_ in path.syn_states if s_[0] == name)
        L1.append(f"{indent}*{syn_ref(path, name)} = {commit_expr(dtype, var)};")
    inputs2 = {k: v for k, v in _event_inputs(plan, path).items() if k not in local}
    prog2 = DeviceProgram(inputs2, L2, f"q{path.index}_", indent=indent, rng=_edge_rng(plan, path))
    for i, statement in enumerate(statements):
        if i not in sequential:
            continue
        for j, name, slot, dtype in crossing:
            if j == i:
                var = prog2.fresh()
                L2.append(f"{indent}const double {var} = reinterpret_cast<const double*>(syn + {slot * 8 * cap})"
                          f"[staged_at];")
                prog2.symbols[name] = (var, dtype)
        prog2.statements([statement])
    for name in path.code["effects"]["writes"]:
        if name in path.post_aliases:
            state = path.post_aliases[name]
            dtype = next(s_[1] for s_ in tgt.states if s_[0] == state)
            L2.append(f"{indent}post_{state} = {commit_expr(dtype, prog2.symbols[name][0])};")
        elif last.get(name) in sequential:
            dtype = next(s_[1] for s_ in path.syn_states if s_[0] == name)
            L2.append(f"{indent}*{syn_ref(path, name)} = {commit_expr(dtype, prog2.symbols[name][0])};")


def _split_bytes(plan: Plan, group: list[PathwayPlan]) -> int:
    """LDS bytes of a split ordered group's crossing values (0: the group is not split)."""
    if counting_group(group) or any(_split_plan(path) is None for path in group):
        return 0
    return max(8, max(_split_crossings(path) for path in group) * 8 * (1 << plan.shape.cap_bits))


def _group_code(plan: Plan, index: int, group: list[PathwayPlan], hist_base: int) -> str:
    src = plan.populations[group[0].source]
    tgt = plan.populations[group[0].target]
    gvals = sorted({d for path in group for d in path.dvals}, reverse=True)
    L: list[str] = []
    L.append(f"struct Group{index} {{")
    count = counting_group(group)
    L.append(f"    static constexpr u32 NP = {len(group)}u, NG = {len(gvals)}u;")
    L.append(f"    static constexpr bool COUNT = {'true' if count else 'false'};")
    L.append(f"    static constexpr u32 HIST_BASE = {hist_base}u;")
    if group[0].event == "spike":
        ring, cnt, ids, small = src.ring, src.buffers["spk_cnt"], src.buffers["spk_ids"], src.buffers["spk_small"]
    else:
        # a custom event's ring of fired neurons (same layout as the spike ring)
        k = next(k for k, (event, _, _) in enumerate(src.custom_events) if event == group[0].event)
        ring, cnt, ids, small = (src.event_rings[k], src.buffers[f"ering_cnt:{k}"], src.buffers[f"ering_ids:{k}"],
                                 src.buffers[f"ering_small:{k}"])
    L.append(f"    static constexpr u32 SRC_N = {src.count}u, SRC_NB = {src.blocks}u, SRC_R = {ring}u;")
    L.append(f"    static constexpr int SRC_CNT = {cnt}, SRC_IDS = {ids}, SRC_SMALL = {small};")
    L.append(f"    static constexpr int DELIVERED = {plan.delivered_buffer}, FAULT = {plan.fault_buffer};")
    L.append(f"    static constexpr u32 PEND_T = {group[0].pending_ticks}u, PEND_TB = {tgt.blocks}u;")
    L.append(f"    static constexpr bool PEND_SOURCES = {'true' if group[0].pending_sources else 'false'};")
    L.append(f"    static constexpr i64 PEND_START = {src.start_tick}LL;")   # the source clock's first tick
    L.append(f"    static constexpr int PEND_OFF = {group[0].buffers.get('pend_off', 0)}, "
             f"PEND = {group[0].buffers.get('pend', 0)};")
    cases = " ".join(f"case {g}: return {v}u;" for g, v in enumerate(gvals))
    L.append(f"    __device__ static u32 gval(u32 g) {{ switch (g) {{ {cases} default: return 0u; }} }}")
    L.append(f"    static constexpr u32 gval_max = {max(gvals)}u;")
    cases = " ".join(f"case {p}: return {path.index}u;" for p, path in enumerate(group))
    L.append(f"    __device__ static u32 path_index(u32 p) {{ switch (p) {{ {cases} default: return 0u; }} }}")
    L.append("    __device__ static void seg_index(u32 id, u32 g, u32 blk, u64* at, bool* ok) {")
    L.append("        (void)g;")
    L.append("        for (u32 p = 0; p < ATLAS_MAX_NP; ++p) { at[p] = 0; ok[p] = false; }")
    for p, path in enumerate(group):
        local = {v: k for k, v in enumerate(path.dvals)}
        mapping = " ".join(f"case {g}: gp = {local[v]}; break;" for g, v in enumerate(gvals) if v in local)
        L.append("        {")
        L.append(f"            const u32 src = id - {path.sstart}u;")
        L.append("            int gp = -1;")
        L.append(f"            switch (g) {{ {mapping} default: break; }}")
        L.append(f"            ok[{p}] = id != 0xFFFFFFFFu && src < {path.scount}u && gp >= 0;")
        L.append(f"            at[{p}] = ((u64)src * {len(path.dvals)}u + (u32)(gp < 0 ? 0 : gp)) * {tgt.blocks + 1}u + blk;")
        L.append("        }")
    L.append("    }")
    cases = " ".join(f"case {p}: return atlas::buf<const u32>(tab, {path.buffers['seg']});" for p, path in enumerate(group))
    L.append("    __device__ static const u32* seg_ptr(const u64* __restrict__ tab, u32 p) {")
    L.append(f"        switch (p) {{ {cases} default: return atlas::buf<const u32>(tab, {group[0].buffers['seg']}); }}")
    L.append("    }")
    cases = " ".join(f"case {p}: return atlas::buf<const u32>(tab, {path.buffers['row_tgt']})[row];"
                     for p, path in enumerate(group))
    L.append("    __device__ static u32 row_target(const u64* __restrict__ tab, u32 p, u32 row) {")
    L.append(f"        switch (p) {{ {cases} default: return 0u; }}")
    L.append("    }")
    # the row of out-edge position k (rows ordered by target keep the positions source-major)
    cases = " ".join(f"case {p}: return atlas::buf<const u32>(tab, {path.buffers['out_row']})[k];"
                     for p, path in enumerate(group) if path.post_major)
    L.append("    __device__ static u32 record_row(const u64* __restrict__ tab, u32 p, u32 k) {")
    L.append("        (void)tab;")
    L.append(f"        switch (p) {{ {cases} default: return k; }}")
    L.append("    }")
    push = push_group(plan, group)
    queue = plan.queues.get(group[0].index)
    L.append(f"    static constexpr bool PUSH = {'true' if push else 'false'};")
    L.append(f"    static constexpr bool QUEUE = {'true' if queue else 'false'};")
    if queue:
        L.append(f"    static constexpr int QCNT = {group[0].buffers['queue_count']}, QBUF = {group[0].buffers['queue']}, "
                 f"QSORT = {group[0].buffers['queue_scratch']};")
        L.append(f"    static constexpr u32 QCAP = {queue['cap']}u;")
    if push or queue:
        items = sum(len(path.dvals) for path in group)
        L.append(f"    static constexpr u32 AR = {push_depth(group)}u, TB = {tgt.blocks}u, ITEMS = {items}u;")
        if push:
            L.append(f"    static constexpr int ARR = {group[0].buffers['arrivals']};")
        L.append("    __device__ static void push_item(const u64* __restrict__ tab, u32 id, u32 i, u32& lo, u32& n, "
                 "u32& code) {")
        L.append("        lo = 0; n = 0; code = 0;")
        first = 0
        for p, path in enumerate(group):
            D = len(path.dvals)
            delays = " ".join(f"case {g}: d = {v}u; break;" for g, v in enumerate(path.dvals))
            L.append(f"        if (i >= {first}u && i < {first + D}u) {{")
            L.append(f"            const u32 src = id - {path.sstart}u, g = i - {first}u;")
            L.append(f"            if (src < {path.scount}u) {{")
            L.append(f"                const atlas::gptr<const u32> seg = atlas::buf<const u32>(tab, {path.buffers['seg']}) + "
                     f"((u64)src * {D}u + g) * {tgt.blocks + 1}u;")
            L.append("                u32 d = 0;")
            L.append(f"                switch (g) {{ {delays} default: break; }}")
            L.append(f"                lo = seg[0]; n = seg[{tgt.blocks}] - lo; code = {p}u | d << 8;")
            L.append("            }")
            L.append("        }")
            first += D
        L.append("    }")
    slots = count and not push and all("slot" in path.buffers and path.index not in plan.slot_fallback
                                       for path in group)
    edge_slots = _edge_slots(plan, group)
    L.append(f"    static constexpr bool SLOTS = {'true' if slots else 'false'};")
    L.append(f"    static constexpr bool EDGE_SLOTS = {'true' if edge_slots else 'false'};")
    if slots or edge_slots:
        # slot of segment `at` = g * (NB + 1) + blk: XCD-major (see atlas_sim_build_slots)
        px = per_xcd(plan)
        wg = f"({tgt.first_block}u + blk)"
        cases = " ".join(
            f"case {p}: return atlas::buf<const uint4>(tab, {path.buffers['slot']}) + 2 * "
            f"((u64)({wg} / {px}u) * {path.scount * len(path.dvals) * px}ull + (at / {tgt.blocks + 1}u) * {px}u + "
            f"{wg} % {px}u);" for p, path in enumerate(group))
        L.append("    __device__ static const uint4* slot_ptr(const u64* __restrict__ tab, u32 p, u64 at, u32 blk) {")
        L.append(f"        switch (p) {{ {cases} default: return atlas::buf<const uint4>(tab, "
                 f"{group[0].buffers['slot']}); }}")
        L.append("    }")
        # pathways with disjoint source ranges: a fired source has at most one slot per block, found
        # without the per-pathway loop or a division (persistent launches, delay group 0)
        ranges = sorted((path.sstart, path.sstart + path.scount) for path in group)
        disjoint = all(a[1] <= b[0] for a, b in zip(ranges, ranges[1:]))
        L.append(f"    static constexpr bool DISJOINT = {'true' if disjoint else 'false'};")
        L.append("    __device__ static const uint4* source_slot(const u64* __restrict__ tab, u32 id, u32 blk, u32& p) {")
        L.append("        p = NP;")
        for k, path in enumerate(group):
            local = {v: i for i, v in enumerate(path.dvals)}
            if gvals[0] not in local:
                continue
            row = f"(u64)(id - {path.sstart}u) * {len(path.dvals)}u + {local[gvals[0]]}u"
            L.append(f"        if (id - {path.sstart}u < {path.scount}u) {{")
            L.append(f"            p = {k}u;")
            L.append(f"            return atlas::buf<const uint4>(tab, {path.buffers['slot']}) + 2 * ((u64)({wg} / {px}u) * "
                     f"{path.scount * len(path.dvals) * px}ull + ({row}) * {px}u + {wg} % {px}u);")
            L.append("        }")
        L.append(f"        return atlas::buf<const uint4>(tab, {group[0].buffers['slot']});")
        L.append("    }")
        # the slot of one pathway (overlapping source ranges: one slot load per pathway)
        L.append("    __device__ static const uint4* source_slot_of(const u64* __restrict__ tab, u32 id, u32 p, u32 blk, "
                 "u32& pq) {")
        L.append("        pq = NP;")
        for k, path in enumerate(group):
            local = {v: i for i, v in enumerate(path.dvals)}
            if gvals[0] not in local:
                continue
            row = f"(u64)(id - {path.sstart}u) * {len(path.dvals)}u + {local[gvals[0]]}u"
            L.append(f"        if (p == {k}u && id - {path.sstart}u < {path.scount}u) {{")
            L.append(f"            pq = {k}u;")
            L.append(f"            return atlas::buf<const uint4>(tab, {path.buffers['slot']}) + 2 * ((u64)({wg} / {px}u) * "
                     f"{path.scount * len(path.dvals) * px}ull + ({row}) * {px}u + {wg} % {px}u);")
            L.append("        }")
        L.append(f"        return atlas::buf<const uint4>(tab, {group[0].buffers['slot']});")
        L.append("    }")
    else:
        L.append("    __device__ static const uint4* slot_ptr(const u64* __restrict__ tab, u32 p, u64 at, u32 blk) "
                 "{ (void)tab; (void)p; (void)at; (void)blk; return nullptr; }")
    post = {}
    written = set()
    for path in group:
        r, w = _touched_post(path)
        for state in (r | w) - {"\0not_refractory"}:
            post[state] = next(s_[1] for s_ in tgt.states if s_[0] == state)
        written |= w
    L.append("    struct Post {")
    for state, dtype in post.items():
        L.append(f"        {CTYPE[dtype]} post_{state};")
    L.append("        int unused_;")
    L.append("    };")
    lds = tgt.lds_states
    L.append("    __device__ static void load_post(const u64* __restrict__ tab, u32 neuron, u32 j, Post& ps, "
             "const byte_t* lds) {")
    L.append("        (void)tab; (void)neuron; (void)j; (void)ps; (void)lds;")
    for state, dtype in post.items():
        if state in lds:
            L.append(f"        ps.post_{state} = reinterpret_cast<const {CTYPE[dtype]}*>(lds + {lds[state]})[j];")
        else:
            L.append(f"        ps.post_{state} = atlas::buf<const {CTYPE[dtype]}>(tab, "
                     f"{tgt.buffers['state:' + state]})[neuron];")
    L.append("    }")
    L.append("    __device__ static void store_post(const u64* __restrict__ tab, u32 neuron, u32 j, const Post& ps, "
             "byte_t* lds) {")
    L.append("        (void)tab; (void)neuron; (void)j; (void)ps; (void)lds;")
    for state, dtype in post.items():
        if state in written:
            if state in lds:
                L.append(f"        reinterpret_cast<{CTYPE[dtype]}*>(lds + {lds[state]})[j] = ps.post_{state};")
            else:
                L.append(f"        atlas::buf<{CTYPE[dtype]}>(tab, {tgt.buffers['state:' + state]})[neuron] = "
                         f"ps.post_{state};")
    L.append("    }")
    cap = 1 << plan.shape.cap_bits
    split = _split_bytes(plan, group) > 0
    staged = None if count or split else _prefetch_layout(plan, group)
    L.append(f"    static constexpr bool PREFETCH = {'true' if staged else 'false'};")
    L.append(f"    static constexpr bool SPLIT = {'true' if split else 'false'};")
    phase1, phase2 = [], []
    if split:
        # fetch: one event's per-edge values into registers; edge_part: the statements of the
        # event's own edge (run for every staged event at once); apply runs the rest in order
        fetches, words = [], 1
        for p, path in enumerate(group):
            lines: list = []
            n, exprs, _ = _register_fetch(path, lines, "            ")
            words = max(words, n)
            fetches.append(lines)
            L1: list = []
            L2: list = []
            _split_code(plan, path, exprs, cap, L1, L2, "                ")
            phase1.append(L1)
            phase2.append(L2)
        L.append(f"    struct Edge {{ u32 w[{words}]; }};")
        L.append("    __device__ static void fetch(const u64* __restrict__ tab, u32 p, u32 row, Edge& v) {")
        L.append("        (void)tab; (void)p; (void)row; (void)v;")
        L.append("        switch (p) {")
        for p, lines in enumerate(fetches):
            L.append(f"        case {p}: {{")
            L.extend(lines)
            L.append("            break;")
            L.append("        }")
        L.append("        default: break;")
        L.append("        }")
        L.append("    }")
        L.append("    __device__ static void stash(const Edge&, u32, u32, byte_t*) {}")
        L.append("    __device__ static void edge_part(const u64* __restrict__ tab, u32 p, u32 row, const Edge& v, u32 at, "
                 "byte_t* syn, double t, i64 tick, u32& fault) {")
        L.append("        (void)tab; (void)row; (void)v; (void)at; (void)syn; (void)t; (void)tick; (void)fault;")
        L.append("        switch (p) {")
        for p, lines in enumerate(phase1):
            L.append(f"        case {p}: {{")
            L.extend(lines)
            L.append("            break;")
            L.append("        }")
        L.append("        default: break;")
        L.append("        }")
        L.append("    }")
    if not split:
        fetches, words, slots = [], 1, []
        for path in group:
            lines: list = []
            n, _, where = _register_fetch(path, lines, "            ") if staged else (0, {}, {})
            words = max(words, n)
            fetches.append(lines)
            slots.append(where)
        L.append(f"    struct Edge {{ u32 w[{words}]; }};")
        L.append("    __device__ static void edge_part(const u64* __restrict__, u32, u32, const Edge&, u32, byte_t*, "
                 "double, i64, u32&) {}")
        # fetch: the per-edge values of one staged event into registers; stash: into the LDS arrays
        L.append("    __device__ static void fetch(const u64* __restrict__ tab, u32 p, u32 row, Edge& v) {")
        L.append("        (void)tab; (void)p; (void)row; (void)v;")
        L.append("        switch (p) {")
        for p, lines in enumerate(fetches):
            L.append(f"        case {p}: {{")
            L.extend(lines)
            L.append("            break;")
            L.append("        }")
        L.append("        default: break;")
        L.append("        }")
        L.append("    }")
        L.append("    __device__ static void stash(const Edge& v, u32 p, u32 at, byte_t* syn) {")
        L.append("        (void)v; (void)p; (void)at; (void)syn;")
        L.append("        switch (p) {")
        for p, mine in enumerate(staged or []):
            L.append(f"        case {p}: {{")
            for name, dtype, offset in mine:
                w = slots[p][name][1]
                if np.dtype(NUMPY[dtype]).itemsize == 8:
                    L.append(f"            reinterpret_cast<u64*>(syn + {offset})[at] = "
                             f"(u64)v.w[{w}] | (u64)v.w[{w + 1}] << 32;")
                else:
                    L.append(f"            reinterpret_cast<u32*>(syn + {offset})[at] = v.w[{w}];")
            L.append("            break;")
            L.append("        }")
        L.append("        default: break;")
        L.append("        }")
        L.append("    }")
    L.append("    __device__ static void apply(const u64* __restrict__ tab, u32 neuron, Post& ps, const u16* keys, "
             "u32 n, const u32* ev_row, const byte_t* syn, double t, i64 tick, u32& fault) {")
    L.append("        (void)tick; (void)t; (void)fault; (void)neuron; (void)syn;")
    for state, dtype in post.items():
        L.append(f"        {CTYPE[dtype]} post_{state} = ps.post_{state};")
    L.append("        for (u32 e = 0; e < n; ++e) {")
    L.append("            const u32 key = keys[e];")
    L.append("            const u32 staged_at = key & (ATLAS_CAP - 1u);")
    L.append("            const u32 row = ev_row[staged_at];")
    L.append("            (void)row; (void)staged_at;")
    L.append("            switch (key >> ATLAS_CAP_BITS) {")
    for p, path in enumerate(group):
        L.append(f"            case {p}: {{")
        lds_values = {name: f"(double)reinterpret_cast<const {CTYPE[dtype]}*>(syn + {offset})[staged_at]"
                      for name, dtype, offset in staged[p]} if staged else None
        if split:
            L.extend(phase2[p])
        else:
            _event_program(plan, path, L, "                ", lds_values)
        L.append("                break;")
        L.append("            }")
    L.append("            default: break;")
    L.append("            }")
    L.append("        }")
    for state in post:
        if state in written:
            L.append(f"        ps.post_{state} = post_{state};")
    L.append("    }")
    if edge_slots:
        L.extend(_edge_group_code(plan, group, post, written))
    if count:
        # counts[p * STRIDE]: the LDS counters (STRIDE = ATLAS_BLOCK) or counts already in registers
        L.append("    template <u32 STRIDE = ATLAS_BLOCK>")
        L.append("    __device__ static void apply_counts(const u64* __restrict__ tab, u32 neuron, Post& ps, "
                 "const u32* counts, double t, i64 tick, u32& fault) {")
        L.append("        (void)tab; (void)tick; (void)t; (void)fault; (void)neuron;")
        for state, dtype in post.items():
            L.append(f"        {CTYPE[dtype]} post_{state} = ps.post_{state};")
        for p, path in enumerate(group):
            body: list = []
            prog = _event_program(plan, path, body, "            ")
            # a post state whose committed value is checked, equals its stored value, and derives
            # from the state's own value through propagating operations: a non-finite value of one
            # event makes every later event's value non-finite, so checking the last event's stored
            # value after the loop raises the same fault at the same tick
            after = []
            for name in path.code["effects"]["writes"]:
                if name not in path.post_aliases:
                    continue
                state = path.post_aliases[name]
                dtype = post[state]
                value = prog.symbols[name][0]
                check = prog.pending.get(value)
                if (check is not None and check[1] is None and name in prog.input_var
                        and (dtype == "f64" or value in prog.rounded32)
                        and prog.propagates(prog.input_var[name], value)):
                    body[check[0]] = f"            // finiteness of {value} checked after the loop"
                    after.append(f"        if (n{p}) atlas::finite((double)post_{state}, fault);")
            L.append(f"        const u32 n{p} = counts[{p}u * STRIDE];")
            L.append(f"        for (u32 e = 0; e < n{p}; ++e) {{")
            L.extend(body)
            L.append("        }")
            L.extend(after)
        for state in post:
            if state in written:
                L.append(f"        ps.post_{state} = post_{state};")
        L.append("    }")
    L.append("};")
    return "\n".join(L)


def _edge_group_code(plan: Plan, group: list[PathwayPlan], post: dict, written: set) -> list[str]:
    """edge_value and apply_edge of an ordered group in the split loop: the per-edge value a
    pathway's program reads (a procedural draw from the edge id, or a load of the row's value),
    computed where the event is listed, and the program of one event given that value."""
    L: list[str] = []
    reads = [[name for name, _ in _edge_values(path)] for path in group]
    L.append("    __device__ static double edge_value(const u64* __restrict__ tab, u32 p, u32 row) {")
    L.append("        (void)tab; (void)p; (void)row;")
    if all(len(r) == 1 and r[0] in path.edge_gen for r, path in zip(reads, group)):
        # every pathway draws a procedural uniform: its constants selected, one draw
        gens = [path.edge_gen[r[0]] for r, path in zip(reads, group)]

        def pick(values, fmt):
            expr = fmt(values[-1])
            for p in range(len(values) - 2, -1, -1):
                expr = f"(p == {p}u ? {fmt(values[p])} : {expr})"
            return expr
        L.append(f"        const u64 seed = {pick([g[0] for g in gens], lambda v: f'{v}ull')};")
        L.append(f"        const u64 stream = {pick([g[1] for g in gens], lambda v: f'{v}ull')};")
        L.append(f"        const double lo = {pick([g[2] for g in gens], hexlit)};")
        L.append(f"        const double hi = {pick([g[3] for g in gens], hexlit)};")
        L.append("        return atlas::edge_uniform(seed, stream, (u64)row, lo, hi);")
    else:
        L.append("        switch (p) {")
        for p, (r, path) in enumerate(zip(reads, group)):
            if r:
                L.append(f"        case {p}: return {_edge_param_expr(path, r[0])};")
        L.append("        default: return 0.0;")
        L.append("        }")
    L.append("    }")
    L.append("    __device__ static void apply_edge(const u64* __restrict__ tab, u32 neuron, Post& ps, u32 p, u32 row, "
             "double value, double t, i64 tick, u32& fault) {")
    L.append("        (void)tab; (void)neuron; (void)row; (void)value; (void)t; (void)tick; (void)fault;")
    for state, dtype in post.items():
        L.append(f"        {CTYPE[dtype]} post_{state} = ps.post_{state};")
    L.append("        switch (p) {")
    for p, (r, path) in enumerate(zip(reads, group)):
        L.append(f"        case {p}: {{")
        _event_program(plan, path, L, "            ", {r[0]: "value"} if r else None)
        L.append("            break;")
        L.append("        }")
    L.append("        default: break;")
    L.append("        }")
    for state in post:
        if state in written:
            L.append(f"        ps.post_{state} = post_{state};")
    L.append("    }")
    return L


def _fused_edge_code(plan: Plan, pop: "PopulationPlan", k: int, group: list[PathwayPlan]) -> str:
    """The split loop's application of one edge-keyed event (key = pathway << EDGE_KEY_BITS | edge
    id, with the per-edge value listed beside it) to a neuron's states in registers."""
    touched, written = {}, set()
    for path in group:
        r, w = _touched_post(path)
        for state in (r | w) - {"\0not_refractory"}:
            touched[state] = True
        written |= w
    L = [f"struct Fused{pop.index} {{",
         f"    __device__ static void apply_edge(const u64* __restrict__ tab, u32 i, Pop{pop.index}::State& st, "
         "u32 key, double value, double t, i64 tick, u32& fault) {",
         f"        Group{k}::Post ps;"]
    for state in touched:
        L.append(f"        ps.post_{state} = st.st_{state};")
    L.append(f"        Group{k}::apply_edge(tab, i, ps, key >> {EDGE_KEY_BITS}u, key & {(1 << EDGE_KEY_BITS) - 1}u, value, "
             "t, tick, fault);")
    for state in touched:
        if state in written:
            L.append(f"        st.st_{state} = ps.post_{state};")
    L.append("    }")
    L.append("};")
    return "\n".join(L)


def _post_code(plan: Plan, post: PostPlan) -> str:
    import dataclasses
    tpop = plan.populations[post.pre.target]
    b = tpop.buffers
    view = dataclasses.replace(post.pre, code=post.code, index=post.index)
    if post.event == "spike":
        ring, cnt, ids = tpop.ring, b["spk_cnt"], b["spk_ids"]
    else:
        # the ring of the target's custom event (published with its spikes)
        k = next(k for k, (event, _, _) in enumerate(tpop.custom_events) if event == post.event)
        ring, cnt, ids = tpop.event_rings[k], b[f"ering_cnt:{k}"], b[f"ering_ids:{k}"]
    L = [f"struct Post{post.index} {{",
         f"    static constexpr u32 N = {tpop.count}u, NB = {tpop.blocks}u, R = {ring}u, D = {post.delay}u, "
         f"NG = {len(post.dvals)}u;",
         "    __device__ static u32 gval(u32 g) { switch (g) { " +
         " ".join(f"case {g}: return {v}u;" for g, v in enumerate(post.dvals)) + " default: return 0u; } }",
         f"    static constexpr u32 TSTART = {post.pre.tstart}u, TCOUNT = {post.pre.tcount}u, INDEX = {post.index}u;",
         f"    static constexpr int CNT = {cnt}, IDS = {ids}, OFF = {post.buffers['off']}, "
         f"ROWS = {post.buffers['rows']}, DELIVERED = {plan.delivered_buffer}, FAULT = {plan.fault_buffer};",
         f"    static constexpr u32 PEND_T = {post.pending_ticks}u;",
         f"    static constexpr bool CONTIGUOUS = {'true' if post.pre.post_major and post.delays is None else 'false'};",
         f"    static constexpr bool PEND_EDGES = {'true' if post.pending is not None and not post.pending[2] else 'false'};",
         f"    static constexpr i64 PEND_START = {tpop.start_tick}LL;",
         f"    static constexpr int PEND_OFF = {post.buffers.get('pend_off', 0)}, PEND = {post.buffers.get('pend', 0)};",
        ]
    # fetch: the per-edge values one event reads, into registers (several events' fetches
    # are issued together); apply: the program on them, stores to memory
    fetch: list = []
    words, exprs, _ = _register_fetch(view, fetch, "        ")
    L.append(f"    struct Edge {{ u32 w[{max(1, words)}]; }};")
    L.append("    __device__ static void fetch(const u64* __restrict__ tab, u32 row, Edge& v) {")
    L.append("        (void)tab; (void)row; (void)v;")
    L.extend(fetch)
    L.append("    }")
    L.append("    __device__ static void apply(const u64* __restrict__ tab, u32 row, const Edge& v, double t, i64 tick, "
             "u32& fault) {")
    L.append("        (void)tab; (void)row; (void)v; (void)t; (void)tick; (void)fault;")
    _event_program(plan, view, L, "        ", exprs)
    L += ["    }", "};"]
    return "\n".join(L)


SYN_WG = 256   # work-items per workgroup of the synapse-code kernels


def _synapse_scalar_env(path: PathwayPlan, dt: float, code: dict) -> dict:
    env = {"dt": dt, "N": float(path.edge_count), "N_pre": float(path.scount), "N_post": float(path.tcount)}
    for name, (_, value) in path.scalar_params.items():
        env[name] = value
    for statement in code["scalar"]:
        value = eval_scalar(statement["value"], env)
        if statement["dtype"] == "f32":
            value = struct.unpack("<f", struct.pack("<f", value))[0]
        env[statement["target"]] = value
    return env


def _synapse_code_kernel(plan: Plan, k: int, code: SynCodePlan) -> tuple[str, int, str]:
    """(kernel name, work-items, source) of one synapse code run before each tick.

    A state update runs one work-item per row: the program on the row's synapse states and
    parameters, its clock-driven states committed (run_synapse_program, executor.rs:2513-2546).
    A summed variable runs one work-item per endpoint neuron: the neuron's edges in edge order,
    each edge's `_synaptic_var` added to a sum that starts at zero, rounded to the state's type
    after every addition as the reference's add_f64 does, and the sum stored
    (run_summed_program, executor.rs:2548-2597)."""
    path = code.path
    b = path.buffers
    tgt = plan.populations[path.target]
    dt = plan.populations[code.population if code.kind == "summed" else path.source].dt
    name = f"atlas_syn{k}"
    if plan.multi_clock:
        # several clocks: the launch is a step of the merged run; the program runs when its own
        # clock advances, at that clock's tick and time (its schedule node's clock)
        c = int(code.code["clock"])
        dt = plan.clocks[c][0]
        L = [f'extern "C" __global__ void __launch_bounds__({SYN_WG}) {name}(const u64* __restrict__ tab, i64 step) {{',
             f"    const i64 tick = atlas::buf<const i64>(tab, {plan.clock_buffer})[(u64)step * {len(plan.clocks)}u + {c}u];",
             "    if (tick < 0) return;",
             f"    const double t = (double)tick * {hexlit(dt)};",
             "    u32 fault = 0;",
             "    (void)t;"]
    else:
        L = [f'extern "C" __global__ void __launch_bounds__({SYN_WG}) {name}(const u64* __restrict__ tab, i64 tick) {{',
             f"    const double t = (double)tick * {hexlit(plan.dt)};",
             "    u32 fault = 0;",
             "    (void)t;"]
    inputs = {"dt": (hexlit(dt), "f64"), "t": ("t", "f64"), "N": (hexlit(float(path.edge_count)), "index"),
              "N_pre": (hexlit(float(path.scount)), "index"), "N_post": (hexlit(float(path.tcount)), "index"),
              "j": (f"(double)(atlas::buf<const u32>(tab, {b.get('row_tgt_rows', b['row_tgt'])})[row] - "
                    f"{path.tstart}u)", "index")}
    for sname, dtype, _ in path.syn_states:
        inputs[sname] = (f"(double)*{syn_ref(path, sname, const=True)}", dtype)
    for pname, (dtype, _) in path.edge_params.items():
        inputs[pname] = (f"atlas::buf<const double>(tab, {b['eparam:' + pname]})[row]", dtype)
    for pname, (dtype, value) in path.scalar_params.items():
        inputs[pname] = (hexlit(value), dtype)
    inputs = _with_scalars(inputs, _synapse_scalar_env(path, dt, code.code), code.code)
    if code.kind == "update":
        units = path.edge_count
        L += [f"    const u32 row = blockIdx.x * {SYN_WG}u + threadIdx.x;",
              f"    if (row >= {units}u) return;"]
        prog = DeviceProgram(inputs, L, "c", indent="    ", rng=_edge_rng(plan, path))
        prog.statements(code.code["vector"])
        for sname in code.code["effects"]["writes"]:
            dtype = next(st[1] for st in path.syn_states if st[0] == sname)
            L.append(f"    *{syn_ref(path, sname)} = {commit_expr(dtype, prog.symbols[sname][0])};")
    else:
        units = code.count
        pop = plan.populations[code.population]
        ct = CTYPE[code.dtype]
        L += [f"    const u32 k = blockIdx.x * {SYN_WG}u + threadIdx.x;",
              f"    if (k >= {units}u) return;",
              f"    const u32 neuron = {code.start}u + k;",
              f"    const u32* off = atlas::buf<const u32>(tab, {code.buffers['off']});",
              f"    const u32* rows = atlas::buf<const u32>(tab, {code.buffers['rows']});",
              f"    {ct} sum = ({ct})0;",
              "    for (u32 p = off[k]; p < off[k + 1]; ++p) {",
              "        const u32 row = rows[p];"]
        if not code.to_pre:
            inputs["j"] = ("(double)k", "index")
            for alias, state in path.post_aliases.items():
                dtype = next(st[1] for st in tgt.states if st[0] == state)
                inputs[alias] = (f"(double)atlas::buf<const {CTYPE[dtype]}>(tab, {tgt.buffers['state:' + state]})"
                                 f"[neuron]", dtype)
        prog = DeviceProgram(inputs, L, "c", indent="        ", rng=_edge_rng(plan, path))
        prog.statements(code.code["vector"])
        value = prog.symbols["_synaptic_var"][0]
        L.append(f"        sum = ({ct})((double)sum + {value});")
        L += ["    }", f"    atlas::buf<{ct}>(tab, {pop.buffers['state:' + code.state]})[neuron] = sum;"]
    L += [f"    atlas::report(tab, {plan.fault_buffer}, fault);", "}"]
    return name, max(1, units), "\n".join(L)


PRELUDE_HELPERS = r"""
namespace atlas {
// Rust `as` conversions of an f64 register to an integer (saturating, NaN -> 0).
__device__ __forceinline__ double saturate_i32(double x) {
    if (!(x == x)) return 0.0;
    if (x >= 2147483647.0) return 2147483647.0;
    if (x <= -2147483648.0) return -2147483648.0;
    return (double)(int)x;
}
__device__ __forceinline__ double saturate_i64(double x) {
    if (!(x == x)) return 0.0;
    return trunc(x);
}
__device__ __forceinline__ double wrap_i32(double x) { return (double)(int)(unsigned int)(long long)x; }
// Counter-based uniform draw (executor.rs:190-222): splitmix64's finaliser (without the
// golden-gamma pre-add) of seed ^ stream C1 ^ tick C2 ^ index C3 (draw 0), top 53 bits.
__device__ __forceinline__ double counter_uniform_draw(u64 seed, u64 stream, u64 tick, u64 index, u64 draw) {
    u64 v = seed ^ (stream * 0x9e3779b97f4a7c15ull) ^ (tick * 0xd1b54a32d192ed03ull) ^ (index * 0x94d049bb133111ebull)
            ^ (draw * 0x369dea0f31a53f85ull);
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    v ^= v >> 31;
    return (double)(v >> 11) * (1.0 / 9007199254740992.0);
}
__device__ __forceinline__ double counter_uniform(u64 seed, u64 stream, u64 tick, u64 index) {
    return counter_uniform_draw(seed, stream, tick, index, 0ull);
}
// Procedural Uniform(lo, hi) value of one edge (large_topology.rs:54-76, 129-142): splitmix64
// with its golden-gamma pre-add of seed ^ stream C1 ^ edge C2 (attempt 0), the top 53 bits plus
// one half scaled to (0, 1), then lo + (hi - lo) u with each operation rounded.
__device__ __forceinline__ double edge_uniform(u64 seed, u64 stream, u64 edge, double lo, double hi) {
    u64 v = (seed ^ (stream * 0xd2b74407b1ce6e93ull) ^ (edge * 0x9e3779b97f4a7c15ull)) + 0x9e3779b97f4a7c15ull;
    v = (v ^ (v >> 30)) * 0xbf58476d1ce4e5b9ull;
    v = (v ^ (v >> 27)) * 0x94d049bb133111ebull;
    v ^= v >> 31;
    const double u = ((double)(v >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    return lo + (hi - lo) * u;
}
// Polar normal of the (index / 2)-th pair, redrawn two draws at a time until the pair lies
// inside the unit disc (executor.rs:200-222).  A draw budget bounds the loop: its end
// (probability (1 - pi/4)^1024) is reported as a fault.
__device__ double counter_normal(u64 seed, u64 stream, u64 tick, u64 index, u32& fault) {
    const u64 pair = index / 2;
    for (u64 draw = 0; draw < 2048; draw += 2) {
        const double x1 = 2.0 * counter_uniform_draw(seed, stream, tick, pair, draw) - 1.0;
        const double x2 = 2.0 * counter_uniform_draw(seed, stream, tick, pair, draw + 1) - 1.0;
        const double radius = x1 * x1 + x2 * x2;
        if (radius < 1.0 && radius != 0.0) {
            const double factor = sqrt(-2.0 * atlas_log(radius) / radius);
            return factor * ((index & 1) == 0 ? x1 : x2);
        }
    }
    fault |= ATLAS_FAULT_RANDOM;
    return 0.0;
}
// Lanczos log-gamma for positive arguments, g = 7, nine terms (executor.rs:270-288).
__device__ double log_gamma_positive(double value) {
    const double c[8] = {676.5203681218851, -1259.1392167224028, 771.3234287776531, -176.6150291621406,
                         12.507343278686905, -0.13857109526572012, 9.984369578019572e-6, 1.5056327351493116e-7};
    const double z = value - 1.0;
    double x = 0.9999999999998099;
    for (int k = 0; k < 8; ++k) x += c[k] / (z + (double)k + 1.0);
    const double t = z + 7.5;
    return 0.9189385332046727 + (z + 0.5) * atlas_log(t) - t + atlas_log(x);
}
// Poisson(lambda) (executor.rs:290-323): the product of uniform draws below lambda = 10, else
// Hormann's transformed rejection (PTRS).  NaN for a rate outside [0, 1e12]; a draw budget
// bounds both loops (its end is reported as a fault).
__device__ double counter_poisson(u64 seed, u64 stream, u64 tick, u64 index, double lambda, u32& fault) {
    if (lambda == 0.0) return 0.0;
    if (!(lambda >= 0.0 && lambda <= 1.0e12)) return __builtin_nan("");
    if (lambda < 10.0) {
        const double limit = atlas_exp(-lambda);
        double product = 1.0;
        for (u64 sample = 0; sample < 4096; ++sample) {
            product *= counter_uniform_draw(seed, stream, tick, index, sample);
            if (product <= limit) return (double)sample;
        }
        fault |= ATLAS_FAULT_RANDOM;
        return 0.0;
    }
    const double root = sqrt(lambda), b = 0.931 + 2.53 * root, a = -0.059 + 0.02483 * b;
    const double inverse_alpha = 1.1239 + 1.1328 / (b - 3.4), squeeze = 0.9277 - 3.6224 / (b - 2.0);
    for (u64 draw = 0; draw < 4096; draw += 2) {
        const double u = counter_uniform_draw(seed, stream, tick, index, draw) - 0.5;
        const double v = counter_uniform_draw(seed, stream, tick, index, draw + 1);
        const double us = 0.5 - fabs(u);
        const double candidate = floor((2.0 * a / us + b) * u + lambda + 0.43);
        if (us >= 0.07 && v <= squeeze) return candidate;
        if (candidate < 0.0 || (us < 0.013 && v > us)) continue;
        const double left = atlas_log(v * inverse_alpha / (a / (us * us) + b));
        const double right = -lambda + candidate * atlas_log(lambda) - log_gamma_positive(candidate + 1.0);
        if (left <= right) return candidate;
    }
    fault |= ATLAS_FAULT_RANDOM;
    return 0.0;
}
// Binomial(n, p) (executor.rs:224-268): the normal approximation when `approximate` and both
// n p and n (1 - p) exceed 5, else inversion from the smaller tail, restarted with the next
// draw past 10 standard deviations (a draw budget bounds the restarts).  An invalid
// probability is a fault (executor.rs:6066-6084).
__device__ double counter_binomial(u64 seed, u64 stream, u64 tick, u64 index, u64 n, double p, bool approximate,
                                   u32& fault) {
    if (!(p >= 0.0 && p <= 1.0)) {
        fault |= ATLAS_FAULT_RANDOM;
        return 0.0;
    }
    if (p <= 0.0) return 0.0;
    if (p >= 1.0) return (double)n;
    const double loc = (double)n * p, complement = (double)n * (1.0 - p);
    if (approximate && loc > 5.0 && complement > 5.0)
        return counter_normal(seed, stream, tick, index, fault) * sqrt(loc * (1.0 - p)) + loc;
    const bool reverse = p > 0.5;
    const double probability = reverse ? 1.0 - p : p, q = 1.0 - probability;
    const double qn = atlas_exp((double)n * atlas_log(q));
    const double bound = fmin((double)n, (double)n * probability + 10.0 * sqrt((double)n * probability * q + 1.0));
    for (u64 draw = 0; draw < 1024; ++draw) {
        u64 x = 0;
        double px = qn;
        double u = counter_uniform_draw(seed, stream, tick, index, draw);
        for (;;) {
            if (u <= px) return reverse ? (double)(n - x) : (double)x;
            x += 1;
            if ((double)x > bound) break;
            u -= px;
            px = ((double)(n - x + 1) * probability * px) / ((double)x * q);
        }
    }
    fault |= ATLAS_FAULT_RANDOM;
    return 0.0;
}
__device__ __forceinline__ double wrap_i64(double x) { return x; }
}  // namespace atlas
"""


def _fused_code(plan: Plan, pop: "PopulationPlan", groups: list) -> str:
    """Apply every counting group's counted events to one neuron's freshly updated states
    (the group's Post view of the State), for phase_a_run."""
    L = [f"struct Fused{pop.index} {{",
         "    template <class L>",
         f"    __device__ static void apply(const u64* __restrict__ tab, u32 i, u32 j, Pop{pop.index}::State& st, "
         "L& s, double t, i64 tick, u32& fault) {",
         "        (void)tab; (void)i; (void)j; (void)st; (void)s; (void)t; (void)tick; (void)fault;"]
    bodies = []
    offset = 0
    for k, group in groups:
        touched, written = {}, set()
        for path in group:
            r, w = _touched_post(path)
            for state in (r | w) - {"\0not_refractory"}:
                touched[state] = True
            written |= w
        bodies.append((k, touched, written, offset))
        offset += len(group)
    for k, touched, written, _ in bodies:
        L.append("        {")
        L.append(f"            Group{k}::Post ps;")
        for state in touched:
            L.append(f"            ps.post_{state} = st.st_{state};")
        L.append(f"            Group{k}::apply_counts(tab, i, ps, &s.hist[Group{k}::HIST_BASE + j], t, tick, fault);")
        for state in touched:
            if state in written:
                L.append(f"            st.st_{state} = ps.post_{state};")
        L.append("        }")
    L.append("    }")
    # the same with each pathway's count given in n[] (the groups' pathways in order), as the
    # split persistent loop reads them from LDS ahead of the applications
    L.append(f"    __device__ static void apply_n(const u64* __restrict__ tab, u32 i, Pop{pop.index}::State& st, "
             "const u32* n, double t, i64 tick, u32& fault) {")
    L.append("        (void)tab; (void)i; (void)st; (void)n; (void)t; (void)tick; (void)fault;")
    for k, touched, written, off in bodies:
        L.append("        {")
        L.append(f"            Group{k}::Post ps;")
        for state in touched:
            L.append(f"            ps.post_{state} = st.st_{state};")
        L.append(f"            Group{k}::template apply_counts<1>(tab, i, ps, n + {off}, t, tick, fault);")
        for state in touched:
            if state in written:
                L.append(f"            st.st_{state} = ps.post_{state};")
        L.append("        }")
    L.append("    }")
    L.append("};")
    return "\n".join(L)


def generate(plan: Plan, header_text: str) -> None:
    """Fill plan.source / kernels / launches (after allocate())."""
    BLOCK, WG, SPT, CAP_BITS = plan.shape.block, plan.shape.wg, plan.shape.spt, plan.shape.cap_bits
    groups = delivery_groups(plan)
    plan.groups = groups
    counting = [counting_group(g) for g in groups]
    post_bytes = 0
    for pop in plan.populations:
        pop.reset_fused = _reset_fusable(plan, pop)
        pop.lds_states = {}
        mine = [k for k, g in enumerate(groups) if g[0].target == pop.index]
        # counted events applied to the states in registers right after the update: every
        # group into the population counts, no on_post pathway waits on the deliveries, and
        # no program reads not_refractory_post (whose `until` the step has not stored yet)
        pop.fused_counts = (not plan.split and bool(mine) and all(counting[k] for k in mine)
                            and not any(post.pre.target == pop.index for post in plan.post_paths)
                            and all("\0not_refractory" not in _touched_post(path)[0]
                                    for k in mine for path in groups[k]))
        # with delay-0 pathways a launch delivers the previous tick, then updates this one: the
        # block's states are loaded first and the previous tick's counted events applied to them
        # in registers before the update, when the same holds and nothing reads the delivered
        # states from memory in between (a reset after the deliveries, PoissonInputs, state
        # monitors)
        pop.fused_split = (plan.split and bool(mine) and all(counting[k] for k in mine)
                           and not any(post.pre.target == pop.index for post in plan.post_paths)
                           and all("\0not_refractory" not in _touched_post(path)[0]
                                   for k in mine for path in groups[k])
                           and (pop.reset is None or pop.reset_fused) and not pop.poisson_inputs
                           and not (pop.monitor_record and pop.monitor_vars) and not pop.custom_events
                           and not any(when == "end" for _, _, _, when in pop.event_monitors))
        if plan.multi_clock:
            # several clocks: a block may receive deliveries at a step that does not update it
            pop.fused_counts = pop.fused_split = False
        # an ordered group through edge-keyed lists, applied in registers by the split loop (the
        # per-tick kernel keeps the ordered LDS path)
        pop.fused_edges = (not plan.split and not plan.multi_clock and len(mine) == 1 and not counting[mine[0]]
                           and _edge_slots(plan, groups[mine[0]]))
        pop.fused_writes = ({state for k in mine for path in groups[k] for state in _touched_post(path)[1]}
                            if pop.fused_counts or pop.fused_split or pop.fused_edges else set())
        if not plan.split and not pop.fused_counts:
            offset = 0
            for path in plan.pathways:
                if path.target != pop.index:
                    continue
                for state in sorted(_touched_post(path)[1]):
                    if state not in pop.lds_states:
                        pop.lds_states[state] = offset
                        dtype = next(s_[1] for s_ in pop.states if s_[0] == state)
                        offset += BLOCK * np.dtype(NUMPY[dtype]).itemsize
            post_bytes = max(post_bytes, offset)
    max_nb = max([plan.populations[g[0].source].blocks for g in groups] + [1])
    max_np = max([len(g) for g in groups] + [1])
    n_delays = lambda g: len({d for path in g for d in path.dvals})  # noqa: E731
    pushing = [push_group(plan, g) for g in groups]
    queued = [g[0].index in plan.queues for g in groups]
    max_gnb = max([n_delays(g) * plan.populations[g[0].source].blocks for k, g in enumerate(groups)
                   if n_delays(g) > 1 and not pushing[k] and not queued[k]] + [1])
    # LDS counter regions: sorting groups share [0, BLOCK); every counting group of a
    # population owns its own region after it, so counts can wait for the update.
    hist_base = [0] * len(groups)
    hist = BLOCK
    for pop in plan.populations:
        mine = [k for k, g in enumerate(groups) if g[0].target == pop.index]
        offset = BLOCK if any(not counting[k] for k in mine) else 0
        for k in mine:
            if counting[k]:
                hist_base[k] = offset
                offset += len(groups[k]) * BLOCK
        hist = max(hist, offset)
    syn_bytes = max([_split_bytes(plan, g) or _prefetch_bytes(plan, g) for k, g in enumerate(groups)
                     if not counting[k]] + [0])
    parts = [f"#define ATLAS_BLOCK {BLOCK}", f"#define ATLAS_WG {WG}", f"#define ATLAS_HIST {hist}",
             f"#define ATLAS_SYN_BYTES {syn_bytes}", f"#define ATLAS_TSTART {BLOCK + 1 if any(queued) else 1}",
             f"#define ATLAS_CAP_BITS {CAP_BITS}", f"#define ATLAS_MAX_NB {max_nb}", f"#define ATLAS_MAX_GNB {max_gnb}",
             f"#define ATLAS_MAX_NP {max_np}", f"#define ATLAS_SPT {SPT}", f"#define ATLAS_POST_BYTES {post_bytes}",
             header_text, PRELUDE_HELPERS]
    for pop in plan.populations:
        parts.append(_population_code(plan, pop))
    for k, group in enumerate(groups):
        parts.append(_group_code(plan, k, group, hist_base[k]))
    for post in plan.post_paths:
        parts.append(_post_code(plan, post))
    for pop in plan.populations:
        if pop.fused_counts or pop.fused_split:
            parts.append(_fused_code(plan, pop, [(k, g) for k, g in enumerate(groups) if g[0].target == pop.index]))
        elif pop.fused_edges:
            k = next(k for k, g in enumerate(groups) if g[0].target == pop.index)
            parts.append(_fused_edge_code(plan, pop, k, groups[k]))
    total = plan.total_blocks
    padded = (total + XCDS - 1) // XCDS * XCDS

    def body(phase_a: bool, phase_b: bool) -> list[str]:
        px = padded // XCDS
        assert px == per_xcd(plan)
        lines = ["    __shared__ atlas::Lds s;", f"    const double t = (double)tick * {hexlit(plan.dt)};",
                 f"    const u32 wg = (blockIdx.x % {XCDS}u) * {px}u + blockIdx.x / {XCDS}u;",
                 f"    if (wg >= {total}u) return;"]
        for pop in plan.populations:
            lines.append(f"    if (wg >= {pop.first_block}u && wg < {pop.first_block + pop.blocks}u) {{")
            lines.append(f"        const u32 blk = wg - {pop.first_block}u;")
            mine = [k for k, g in enumerate(groups) if g[0].target == pop.index]
            deliver = (lambda k, apply, hook="": (
                # a continuation's pending events of an ordered group go first (counting groups
                # add theirs to the counters)
                (f"        atlas::deliver_pending<Group{k}>(tab, tick, t, blk, wg, {total}u, s);\n"
                 if groups[k][0].pending_ticks and not counting[k] else "") + (
                    f"        atlas::take_counts<Group{k}>(tab, tick, blk, wg, {total}u, s{hook});" +
                    (f"\n        atlas::apply_counts<Group{k}>(tab, tick, t, blk, s);\n        __syncthreads();"
                     if apply else "") if pushing[k] else
                    f"        atlas::take_events<Group{k}>(tab, tick, t, blk, wg, {total}u, s);" if queued[k] else
                    f"        atlas::deliver<Group{k}{'' if apply else ', false'}>"
                    f"(tab, tick, t, blk, wg, {total}u, {plan.start_tick}LL, s{hook});")))
            # push and queued groups fed by this population: its spikes of the tick, once published
            producers = [f"        atlas::{'push_counts' if pushing[k] else 'push_events'}<Group{k}>(tab, tick, blk, s);"
                         for k, g in enumerate(groups) if (pushing[k] or queued[k]) and g[0].source == pop.index]
            if producers:
                producers = ["        __threadfence_block();", "        __syncthreads();"] + producers + \
                    ["        __syncthreads();"]
            if phase_a and phase_b and pop.fused_counts:
                # count the tick's events while the state loads are in flight; the update and
                # threshold run inside the first group's counting, under its slot-load latency;
                # then the counted events are applied to the states in registers
                n = pop.index
                lines.append(f"        Pop{n}::State st[ATLAS_ROUNDS];")
                lines.append("        u64 masks[ATLAS_ROUNDS];")
                lines.append("        u32 fault = 0;")
                lines.append(f"        atlas::phase_a_load<Pop{n}>(tab, blk, st);")
                lines.append(f"        const auto step = [&]() {{ atlas::phase_a_step<Pop{n}>(tab, tick, t, blk, st, s, "
                             "masks, fault); };")
                for position, k in enumerate(mine):
                    lines.append(deliver(k, False, ", step" if position == 0 else ""))
                lines.append(f"        atlas::phase_a_finish<Pop{n}, Fused{n}>(tab, tick, t, blk, st, s, masks, fault);")
                lines.append("        __syncthreads();")
                lines.extend(producers)
            elif phase_a and phase_b and any(counting[k] for k in mine):
                # count the tick's events (they depend only on earlier ticks' spikes) while
                # the block's state loads are in flight, then update, then apply in order
                lines.append(f"        Pop{pop.index}::State st[ATLAS_ROUNDS];")
                lines.append(f"        atlas::phase_a_load<Pop{pop.index}>(tab, blk, st);")
                for k in mine:
                    if counting[k]:
                        lines.append(deliver(k, False))
                lines.append(f"        atlas::phase_a_run<Pop{pop.index}>(tab, tick, t, blk, st, s);")
                lines.append("        __syncthreads();")
                lines.extend(producers)
                for k in mine:
                    if counting[k]:
                        lines.append(f"        atlas::apply_counts<Group{k}>(tab, tick, t, blk, s);")
                        lines.append("        __syncthreads();")
                    else:
                        lines.append(deliver(k, True))
                lines.append("        __syncthreads();")
            else:
                if phase_a:
                    lines.append(f"        atlas::phase_a<Pop{pop.index}>(tab, tick, t, blk, s);")
                    lines.extend(producers)
                if phase_b:
                    lines.append("        __syncthreads();")
                    for k in mine:
                        lines.append(deliver(k, True))
                    lines.append("        __syncthreads();")
            posts = [post for post in plan.post_paths if post.pre.target == pop.index]
            if phase_b and posts:
                # on_post pathways run after every on_pre delivery of the tick; spikes of
                # this tick were published by this workgroup's phase A
                lines.append("        __threadfence_block();")
                lines.append("        __syncthreads();")
                for post in posts:
                    if post.pending_ticks:
                        lines.append(f"        atlas::deliver_post_pending<Post{post.index}>(tab, tick, t, blk, wg, "
                                     f"{total}u, s);")
                    lines.append(f"        atlas::deliver_post<Post{post.index}>(tab, tick, t, blk, wg, {total}u, "
                                 f"{plan.start_tick}LL, s);")
                lines.append("        __syncthreads();")
            if phase_b:
                if pop.lds_states:
                    lines.append(f"        atlas::writeback<Pop{pop.index}>(tab, blk, s);")
                    lines.append("        __syncthreads();")
                if pop.poisson_inputs:
                    # after every delivery into the block (written back); an on_post program reads
                    # none of the states they write, so the order against on_post does not matter
                    lines.append(f"        atlas::poisson_phase<Pop{pop.index}>(tab, tick, t, blk);")
                    lines.append("        __threadfence_block();")
                    lines.append("        __syncthreads();")
                lines.append(f"        atlas::reset_phase<Pop{pop.index}>(tab, tick, t, blk);")
                if any(where == "end" for _, where in pop.regular):
                    lines.append("        __threadfence_block();")
                    lines.append("        __syncthreads();")
                    lines.append(f"        atlas::regular_phase<Pop{pop.index}>(tab, tick, t, blk);")
            lines.append("        return;")
            lines.append("    }")
        return lines

    def sections(lines: list[str]) -> dict:
        """The statements of each population's section of a body, by its first line."""
        out, current = {}, None
        for line in lines:
            if line.startswith("    if (wg >= ") and line.endswith("{"):
                current = line
                out[current] = []
            elif line == "    }":
                current = None
            elif current is not None and not line.strip().startswith("const u32 blk =") and line.strip() != "return;":
                out[current].append(line)
        return out

    def shifted_body() -> list[str]:
        # a delay-0 pathway needs every block's spikes of the tick before its deliveries: each
        # launch first delivers the previous tick (whose update the previous launch finished
        # on every block), then updates this tick; the epilogue delivers the run's last tick
        import re
        update, deliver = body(True, False), body(False, True)
        b_sections = sections(deliver)
        lines = update[:4]
        for head, a_lines in sections(update).items():
            lines.append(head)
            lines.append(f"        const u32 blk = wg - {head.split('wg >= ')[1].split('u')[0]}u;")
            first_block = int(head.split('wg >= ')[1].split('u')[0])
            pop = next(p_ for p_ in plan.populations if p_.first_block == first_block)
            if pop.fused_split:
                n = pop.index
                mine = [k for k, g in enumerate(groups) if g[0].target == pop.index]
                lines.append(f"        Pop{n}::State st[ATLAS_ROUNDS];")
                lines.append(f"        atlas::phase_a_load<Pop{n}>(tab, blk, st);")
                lines.append(f"        if (tick > {plan.start_tick}LL) {{")
                lines.append("            const i64 tick_prev = tick - 1;")
                lines.append(f"            const double t_prev = (double)tick_prev * {hexlit(plan.dt)};")
                for k in mine:
                    lines.append(f"            atlas::deliver<Group{k}, false>(tab, tick_prev, t_prev, blk, wg, "
                                 f"{total}u, {plan.start_tick}LL, s);")
                lines.append("            __syncthreads();")
                lines.append(f"            atlas::pre_apply<Pop{n}, Fused{n}>(tab, tick_prev, t_prev, blk, st, s);")
                lines.append("        }")
                lines.append("        __syncthreads();")
                lines.append(f"        atlas::phase_a_run<Pop{n}>(tab, tick, t, blk, st, s);")
                lines.append("        return;")
                lines.append("    }")
                continue
            lines.append(f"        if (tick > {plan.start_tick}LL) {{")
            lines.append("            const i64 tick_prev = tick - 1;")
            lines.append(f"            const double t_prev = (double)tick_prev * {hexlit(plan.dt)};")
            for line in b_sections.get(head, []):
                line = re.sub(r"\btick\b", "tick_prev", line)
                lines.append("    " + re.sub(r"\bt\b", "t_prev", line))
            lines.append("        }")
            lines.append("        __syncthreads();")
            lines.extend(a_lines)
            lines.append("        return;")
            lines.append("    }")
        return lines

    def previous_body() -> list[str]:
        # delay-0 pathways with synapse programs in the groups slot or end-of-tick run_regularly
        # code: the deliveries, resets and end code of the previous tick in a launch of their own,
        # so that the synapse programs of this tick run after them and before this tick's update
        # (the order of the reference's schedule)
        import re
        deliver = body(False, True)
        lines = deliver[:4]
        for head, b_lines in sections(deliver).items():
            lines.append(head)
            lines.append(f"        const u32 blk = wg - {head.split('wg >= ')[1].split('u')[0]}u;")
            lines.append(f"        if (tick > {plan.start_tick}LL) {{")
            lines.append("            const i64 tick_prev = tick - 1;")
            lines.append(f"            const double t_prev = (double)tick_prev * {hexlit(plan.dt)};")
            for line in b_lines:
                line = re.sub(r"\btick\b", "tick_prev", line)
                lines.append("    " + re.sub(r"\bt\b", "t_prev", line))
            lines.append("        }")
            lines.append("        return;")
            lines.append("    }")
        return lines

    def multi_body(part: str = "all") -> list[str]:
        # several clocks: launch `tick` is a step of the merged run.  The clock table gives each
        # clock's tick at it, or -1 where that clock does not advance.  A population's update,
        # threshold, on_post pathways, PoissonInputs and reset run when its clock advances; a
        # delivery group runs when its source's clock does, at the source's tick (its delays
        # and spike ring count the source's ticks).  With delay-0 pathways a step's deliveries
        # need every block's spikes of the step: `part` "a" is the updates (and pushes), "b" the
        # deliveries, on_post pathways, PoissonInputs, resets and end code, in two launches.
        px = padded // XCDS
        C = len(plan.clocks)
        lines = ["    __shared__ atlas::Lds s;",
                 f"    const u32 wg = (blockIdx.x % {XCDS}u) * {px}u + blockIdx.x / {XCDS}u;",
                 f"    if (wg >= {total}u) return;",
                 f"    const i64* __restrict__ clock_ticks = atlas::buf<const i64>(tab, {plan.clock_buffer}) + "
                 f"(u64)tick * {C}u;"]
        for c, (dt_c, _, _) in enumerate(plan.clocks):
            lines.append(f"    const i64 tick{c} = clock_ticks[{c}];")
            lines.append(f"    const double t{c} = (double)tick{c} * {hexlit(dt_c)};")
        for pop in plan.populations:
            c, n = pop.clock, pop.index
            mine = [k for k, g in enumerate(groups) if g[0].target == n]
            lines.append(f"    if (wg >= {pop.first_block}u && wg < {pop.first_block + pop.blocks}u) {{")
            lines.append(f"        const u32 blk = wg - {pop.first_block}u;")
            if part != "b":
                lines.append(f"        if (tick{c} >= 0) {{")
                lines.append(f"            atlas::phase_a<Pop{n}>(tab, tick{c}, t{c}, blk, s);")
                producers = [f"            atlas::{'push_counts' if pushing[k] else 'push_events'}<Group{k}>"
                             f"(tab, tick{c}, blk, s);"
                             for k, g in enumerate(groups) if (pushing[k] or queued[k]) and g[0].source == n]
                if producers:
                    lines.extend(["            __threadfence_block();", "            __syncthreads();"] + producers +
                                 ["            __syncthreads();"])
                lines.append("        }")
            if part == "a":
                lines.append("        return;")
                lines.append("    }")
                continue
            source_clocks = sorted({plan.populations[groups[k][0].source].clock for k in mine})
            others = [sc for sc in source_clocks if sc != c]
            if others and pop.lds_states:
                cond = " || ".join(f"tick{sc} >= 0" for sc in others)
                lines.append(f"        else if ({cond}) atlas::stage<Pop{n}>(tab, blk, s);")
            if mine:
                lines.append("        __syncthreads();")
                for k in mine:
                    sc = plan.populations[groups[k][0].source].clock
                    start = plan.clocks[sc][1]
                    lines.append(f"        if (tick{sc} >= 0) {{")
                    if groups[k][0].pending_ticks and not counting[k]:
                        # a continuation's pending events of an ordered group go first
                        lines.append(f"            atlas::deliver_pending<Group{k}>(tab, tick{sc}, t{sc}, blk, wg, "
                                     f"{total}u, s);")
                    if pushing[k]:
                        lines.append(f"            atlas::take_counts<Group{k}>(tab, tick{sc}, blk, wg, {total}u, s);")
                        lines.append(f"            atlas::apply_counts<Group{k}>(tab, tick{sc}, t{sc}, blk, s);")
                        lines.append("            __syncthreads();")
                    elif queued[k]:
                        lines.append(f"            atlas::take_events<Group{k}>(tab, tick{sc}, t{sc}, blk, wg, "
                                     f"{total}u, s);")
                    else:
                        lines.append(f"            atlas::deliver<Group{k}>(tab, tick{sc}, t{sc}, blk, wg, {total}u, "
                                     f"{start}LL, s);")
                    lines.append("        }")
                lines.append("        __syncthreads();")
            posts = [post for post in plan.post_paths if post.pre.target == n]
            if posts:
                lines.append(f"        if (tick{c} >= 0) {{")
                lines.append("            __threadfence_block();")
                lines.append("            __syncthreads();")
                for post in posts:
                    if post.pending_ticks:
                        lines.append(f"            atlas::deliver_post_pending<Post{post.index}>(tab, tick{c}, t{c}, "
                                     f"blk, wg, {total}u, s);")
                    lines.append(f"            atlas::deliver_post<Post{post.index}>(tab, tick{c}, t{c}, blk, wg, "
                                 f"{total}u, {plan.clocks[c][1]}LL, s);")
                lines.append("            __syncthreads();")
                lines.append("        }")
            if pop.lds_states:
                cond = " || ".join(f"tick{sc} >= 0" for sc in sorted({c} | set(source_clocks)))
                lines.append(f"        if ({cond}) {{")
                lines.append(f"            atlas::writeback<Pop{n}>(tab, blk, s);")
                lines.append("            __syncthreads();")
                lines.append("        }")
            lines.append(f"        if (tick{c} >= 0) {{")
            if pop.poisson_inputs:
                lines.append(f"            atlas::poisson_phase<Pop{n}>(tab, tick{c}, t{c}, blk);")
                lines.append("            __threadfence_block();")
                lines.append("            __syncthreads();")
            lines.append(f"            atlas::reset_phase<Pop{n}>(tab, tick{c}, t{c}, blk);")
            if any(where == "end" for _, where in pop.regular):
                lines.append("            __threadfence_block();")
                lines.append("            __syncthreads();")
                lines.append(f"            atlas::regular_phase<Pop{n}>(tab, tick{c}, t{c}, blk);")
            lines.append("        }")
            lines.append("        return;")
            lines.append("    }")
        return lines

    def persistent_body() -> list[str]:
        # one cooperative launch runs `ticks` ticks: the block's states stay in registers, the
        # spike ring is exchanged device-coherently and a grid barrier separates the ticks
        pop = plan.populations[0]
        px = padded // XCDS
        n = pop.index
        mine = [k for k, g in enumerate(groups) if g[0].target == pop.index]
        assert len(mine) == 1
        if split_loop:
            # delay >= 1: exchange and update waves side by side (atlas_tick.h persistent_run_split)
            return ["    __shared__ atlas::LdsSplit s;",
                    f"    const u32 wg = (blockIdx.x % {XCDS}u) * {px}u + blockIdx.x / {XCDS}u;",
                    f"    if (wg >= {total}u) return;",
                    f"    atlas::persistent_run_split<Pop{n}, Group{mine[0]}, Fused{n}>(tab, tick0, ticks, wg, {total}u, "
                    f"{plan.start_tick}LL, {hexlit(plan.dt)}, s);"]
        return ["    __shared__ atlas::Lds s;",
                f"    const u32 wg = (blockIdx.x % {XCDS}u) * {px}u + blockIdx.x / {XCDS}u;",
                f"    if (wg >= {total}u) return;",
                f"    atlas::persistent_run<Pop{n}, Group{mine[0]}, Fused{n}>(tab, tick0, ticks, wg, {total}u, "
                f"{plan.start_tick}LL, {hexlit(plan.dt)}, {plan.barrier_buffer}, s);"]

    plan.epilogue = []
    # delay 0 with synapse programs in the groups slot or run_regularly code at the end of the tick:
    # the previous tick's deliveries, resets and end code in a launch before this tick's
    separate = plan.split and not plan.multi_clock and (
        plan.synapse_codes or any(where == "end" for pop in plan.populations for _, where in pop.regular))
    if separate:
        kernels = [("atlas_tick", body(True, False)), ("atlas_tick_deliver", body(False, True)),
                   ("atlas_tick_deliver_previous", previous_body())]
        plan.epilogue = [(1, padded, WG, 0)]
    elif plan.multi_clock and plan.split:
        kernels = [("atlas_tick", multi_body("a")), ("atlas_tick_deliver", multi_body("b"))]
    elif plan.split:
        kernels = [("atlas_tick", shifted_body()), ("atlas_tick_deliver", body(False, True))]
        plan.epilogue = [(1, padded, WG, 0)]
    elif plan.multi_clock:
        kernels = [("atlas_tick", multi_body())]
    else:
        kernels = [("atlas_tick", body(True, True))]
    for name, lines in kernels:
        parts.append(f'extern "C" __global__ void __launch_bounds__({WG}) {name}(const u64* __restrict__ tab, i64 tick) {{')
        parts.extend(lines)
        parts.append("}")
    plan.persistent = None
    # the split loop needs a delay of at least one tick, two halves of waves and at most 64 source
    # blocks per exchange wave (the first exchange wave only publishes)
    xwaves = SPLIT_XWAVES or WG // 128
    # and one fired mask per lane of the publishing wave: (rounds per update work-item) x (update waves)
    split_loop = (PERSISTENT_SPLIT and not plan.split and 1 <= xwaves < WG // 64
                  and plan.total_blocks <= 64 * max(1, xwaves - 1)
                  and -(-BLOCK // (WG - 64 * xwaves)) * (WG // 64 - xwaves) <= 64)
    if split_loop:
        parts.insert(parts.index(header_text), f"#define ATLAS_XWAVES {xwaves}u")
    eligible = persistent_eligible(plan, groups, counting, split_loop)
    if eligible and split_loop and plan.populations[0].fused_edges:
        # the edge buckets take the LDS the split loop's other arrays leave (LdsSplit), by tick
        # parity: a count array of BLOCK + 4 words, a key (4 bytes) and a value (8 bytes) per event;
        # the fired lists are shortened to EDGE_XLIST entries per wave (longer ones read the ring)
        fixed = (4 * 64 + 24 + 8 * 64 + 4 * 2 * (WG // 64) * max_np + 16
                 + 4 * EDGE_XLIST * xwaves + 4 * 64 * xwaves + 256)
        words = (LDS_BYTES - fixed) // 4
        counts = BLOCK + BLOCK // 64 + 4     # one pad word per 64 counts (atlas_tick.h edge_at)
        nodes = (words - 2 * counts) // 6 // 2 * 2
        parts.insert(parts.index(header_text), f"#define ATLAS_XLIST {EDGE_XLIST}u")
        parts.insert(parts.index(header_text), f"#define ATLAS_SPLIT_HIST {2 * counts + 6 * nodes}u")
        parts.insert(parts.index(header_text), f"#define ATLAS_EDGE_NODES {nodes}u")
        plan.edge_nodes = nodes
    if eligible:
        # every workgroup must be resident at once: the waves per SIMD the grid needs (two 512-wide
        # workgroups per CU for 489 blocks of 2048: 4, at most 128 VGPRs; one 1024-wide for 245 of 4096:
        # 4; one 256-wide for configs 1 and 2: 1, so config 2's HH update keeps its values in registers)
        waves = max(1, -(-plan.total_blocks // CUS) * (WG // 64) // 4)
        parts.append(f'extern "C" __global__ void __launch_bounds__({WG}) __attribute__((amdgpu_waves_per_eu({waves}))) '
                     "atlas_run(const u64* __restrict__ tab, i64 tick0, i64 ticks) {")
        parts.extend(persistent_body())
        parts.append("}")
        plan.persistent = (len(kernels), padded, WG, 0)
        kernels.append(("atlas_run", []))
    # synapse state updates and summed variables, each its own launch before the tick kernel,
    # in schedule order
    pre_tick = []
    for k, code in enumerate(plan.synapse_codes):
        name, units, text = _synapse_code_kernel(plan, k, code)
        parts.append(text)
        pre_tick.append((len(kernels), (units + SYN_WG - 1) // SYN_WG, SYN_WG, 0))
        kernels.append((name, []))
    plan.source = "\n".join(parts) + "\n"
    plan.kernels = [name for name, _ in kernels]
    plan.launches = pre_tick + [(0, padded, WG, 0)]
    if separate:
        plan.launches = [(2, padded, WG, 0)] + plan.launches
    elif plan.multi_clock and plan.split:
        plan.launches.append((1, padded, WG, 0))


COMPILE_OPTIONS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-ffp-contract=off", "-fno-fast-math",
                   "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
