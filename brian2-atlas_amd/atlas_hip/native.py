"""ctypes binding of ``libatlas_sim_hip.so`` (C ABI in ``include/atlas_sim.h``).

The library is built in-tree by ``__graft_entry__.build()``.  There is no CPU
fallback: every entry point raises ``NativeUnavailable`` when the library is
missing, and ``NativeError`` (carrying the ABI return code) when a call fails.
"""
from __future__ import annotations

import atexit
import ctypes
import os
import weakref
from pathlib import Path

import numpy as np

PACKAGE_ROOT = Path(__file__).resolve().parent.parent
LIBRARY = PACKAGE_ROOT / "libatlas_sim_hip.so"
DEVICE_HEADER = PACKAGE_ROOT / "csrc" / "device" / "atlas_tick.h"
MATH_HEADER = PACKAGE_ROOT / "csrc" / "device" / "atlas_math.h"
MATH_TABLES = PACKAGE_ROOT / "csrc" / "device" / "atlas_math_tables.h"


def device_header_text() -> str:
    """The hand-written device sources prepended to every generated module: the
    shared exponential (tables inlined, since hiprtc compiles a single string) and
    the tick templates."""
    return "\n".join([MATH_TABLES.read_text(), "#define ATLAS_MATH_TABLES_INLINED 1", MATH_HEADER.read_text(),
                      DEVICE_HEADER.read_text()])

CODES = {1: "device", 2: "alloc", 3: "upload", 4: "kernel", 5: "readback", 6: "compile", 7: "host", 8: "cooperative"}
COOPERATIVE = 8   # ATLAS_E_COOPERATIVE: a persistent grid cannot be resident at once
PERSISTENT_PLAIN = 1   # atlas_sim.h ATLAS_PERSISTENT_PLAIN


class NativeUnavailable(RuntimeError):
    """libatlas_sim_hip.so is not built; the HIP engine has no fallback."""


class NativeError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"atlas_sim [{CODES.get(code, code)}]: {message}")
        self.code = code


class Launch(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_uint32), ("grid_x", ctypes.c_uint32), ("block_x", ctypes.c_uint32),
                ("shared_bytes", ctypes.c_uint32)]


class RunStats(ctypes.Structure):
    _fields_ = [("device_seconds", ctypes.c_double), ("host_seconds", ctypes.c_double),
                ("ticks", ctypes.c_int64), ("launches", ctypes.c_uint64)]


class FixedIndegree(ctypes.Structure):
    _fields_ = [("source_count", ctypes.c_uint64), ("target_count", ctypes.c_uint64),
                ("indegree", ctypes.c_uint64), ("seed", ctypes.c_uint64),
                ("target_start", ctypes.c_uint64), ("block", ctypes.c_uint64), ("blocks", ctypes.c_uint64),
                ("row_target_buffer", ctypes.c_uint32), ("segment_buffer", ctypes.c_uint32)]


class SlotTable(ctypes.Structure):
    _fields_ = [("segment_buffer", ctypes.c_uint32), ("row_target_buffer", ctypes.c_uint32),
                ("slot_buffer", ctypes.c_uint32), ("block", ctypes.c_uint32), ("groups", ctypes.c_uint64),
                ("blocks", ctypes.c_uint64), ("first_block", ctypes.c_uint64), ("per_xcd", ctypes.c_uint64),
                ("xcds", ctypes.c_uint64), ("row_slots", ctypes.c_uint32)]


EXPORTS = ["atlas_sim_create", "atlas_sim_destroy", "atlas_sim_alloc", "atlas_sim_upload", "atlas_sim_read",
           "atlas_sim_zero", "atlas_sim_copy", "atlas_sim_compile", "atlas_sim_set_schedule", "atlas_sim_run",
           "atlas_sim_fixed_indegree", "atlas_sim_build_slots", "atlas_sim_extract_spikes", "atlas_sim_set_profiling",
           "atlas_sim_kernel_time", "atlas_sim_set_epilogue", "atlas_sim_device_name", "atlas_sim_set_persistent",
           "atlas_prepare_fixed_indegree", "atlas_prepare_fixed_total", "atlas_prepare_initializer"]

_lib = None


def library() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists():
        raise NativeUnavailable(f"{LIBRARY} is not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIBRARY))
    e = (ctypes.c_char_p, ctypes.c_size_t)
    vp, u32, u64, i64 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_int64
    lib.atlas_sim_create.argtypes = [ctypes.c_int, ctypes.POINTER(vp), *e]
    lib.atlas_sim_destroy.argtypes = [vp]
    lib.atlas_sim_destroy.restype = None
    lib.atlas_sim_alloc.argtypes = [vp, u64, vp, ctypes.POINTER(u32), *e]
    lib.atlas_sim_upload.argtypes = [vp, u32, u64, vp, u64, *e]
    lib.atlas_sim_read.argtypes = [vp, u32, u64, vp, u64, *e]
    lib.atlas_sim_zero.argtypes = [vp, u32, u64, u64, *e]
    lib.atlas_sim_copy.argtypes = [vp, u32, u64, u32, u64, u64, *e]
    lib.atlas_sim_compile.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), u32,
                                      ctypes.POINTER(ctypes.c_char_p), u32, *e]
    lib.atlas_sim_set_schedule.argtypes = [vp, ctypes.POINTER(Launch), u32, *e]
    lib.atlas_sim_set_epilogue.argtypes = [vp, ctypes.POINTER(Launch), u32, *e]
    lib.atlas_sim_run.argtypes = [vp, i64, i64, ctypes.POINTER(RunStats), *e]
    lib.atlas_sim_fixed_indegree.argtypes = [vp, ctypes.POINTER(FixedIndegree), *e]
    lib.atlas_sim_build_slots.argtypes = [vp, ctypes.POINTER(SlotTable), ctypes.POINTER(u32), *e]
    lib.atlas_sim_extract_spikes.argtypes = [vp, u32, u64, u64, u64, vp, u64, ctypes.POINTER(u64), *e]
    lib.atlas_sim_set_profiling.argtypes = [vp, ctypes.c_int, *e]
    lib.atlas_sim_kernel_time.argtypes = [vp, u32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(u64), *e]
    lib.atlas_sim_device_name.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t, *e]
    lib.atlas_sim_set_persistent.argtypes = [vp, ctypes.POINTER(Launch), u32, i64, u32, *e]
    u32p, f64p = ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_double)
    lib.atlas_prepare_fixed_indegree.argtypes = [u64, u64, u64, u64, u32p, u32p, *e]
    lib.atlas_prepare_fixed_total.argtypes = [u64, u64, u64, u64, u32p, u32p, *e]
    lib.atlas_prepare_initializer.argtypes = [ctypes.c_int, u64, u64, u64, ctypes.c_double, ctypes.c_double,
                                              ctypes.c_double, ctypes.c_double, ctypes.c_int, ctypes.c_int, f64p, *e]
    for name in EXPORTS:
        if name != "atlas_sim_destroy":
            getattr(lib, name).restype = ctypes.c_int
    _lib = lib
    return lib


def _check(rc: int, err) -> None:
    if rc != 0:
        raise NativeError(rc, err.value.decode(errors="replace"))


class PrepareError(ValueError):
    """An invalid procedural topology or initializer specification (the reference's message)."""


def _prepare(name: str, *args) -> None:
    err = ctypes.create_string_buffer(1024)
    if getattr(library(), name)(*args, err, len(err)) != 0:
        raise PrepareError(err.value.decode(errors="replace"))


def prepare_fixed_indegree(sources: int, targets: int, indegree: int, seed: int):
    """(source, target) u32 arrays of a fixed-in-degree rule in the reference's order, on the host."""
    import numpy as np
    n = max(0, targets * indegree)
    src, tgt = np.empty(n, np.uint32), np.empty(n, np.uint32)
    u32p = ctypes.POINTER(ctypes.c_uint32)
    _prepare("atlas_prepare_fixed_indegree", sources, targets, indegree, seed & (2**64 - 1),
             src.ctypes.data_as(u32p), tgt.ctypes.data_as(u32p))
    return src, tgt


def prepare_fixed_total(sources: int, targets: int, edges: int, seed: int):
    """(source, target) u32 arrays of a fixed-total rule in the reference's order, on the host."""
    import numpy as np
    src, tgt = np.empty(max(0, edges), np.uint32), np.empty(max(0, edges), np.uint32)
    u32p = ctypes.POINTER(ctypes.c_uint32)
    _prepare("atlas_prepare_fixed_total", sources, targets, edges, seed & (2**64 - 1),
             src.ctypes.data_as(u32p), tgt.ctypes.data_as(u32p))
    return src, tgt


def prepare_initializer(kind: int, count: int, seed: int, stream: int, minimum: float = 0.0, maximum: float = 0.0,
                        mean: float = 0.0, std: float = 0.0, has_minimum: bool = True, has_maximum: bool = True):
    """Per-edge initializer values (0 uniform, 1 clipped normal) on the host, f64."""
    import numpy as np
    out = np.empty(count, np.float64)
    _prepare("atlas_prepare_initializer", kind, count, seed & (2**64 - 1), stream, minimum, maximum, mean, std,
             int(has_minimum), int(has_maximum), out.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    return out


# Every open device handle (simulations here, trainers in rsnn.py) is closed explicitly when the
# interpreter exits, before the C runtime's exit handlers: the HIP module, stream and buffers are
# then released while the HIP runtime (and a profiler attached to it) is still up, never by a
# destructor running after they have finalised.
_open_handles: "weakref.WeakSet" = weakref.WeakSet()


def track(handle_owner) -> None:
    """Register an object with a close() method for the explicit teardown at exit."""
    _open_handles.add(handle_owner)


@atexit.register
def close_all() -> None:
    for owner in list(_open_handles):
        try:
            owner.close()
        except Exception:
            pass


class Sim:
    """One resident simulation on one device."""

    def __init__(self, device: int | None = None):
        self._lib = library()
        if device is None:
            device = int(os.environ.get("B2_SIM_HIP_DEVICE", "0"))
        self._err = ctypes.create_string_buffer(8192)
        handle = ctypes.c_void_p()
        _check(self._lib.atlas_sim_create(device, ctypes.byref(handle), self._err, len(self._err)), self._err)
        self._handle = handle
        self.sizes: list[int] = []
        track(self)

    def _call(self, name: str, *args) -> None:
        _check(getattr(self._lib, name)(self._handle, *args, self._err, len(self._err)), self._err)

    def alloc(self, nbytes: int, init: np.ndarray | bytes | None = None) -> int:
        buffer = ctypes.c_uint32()
        if init is None:
            self._call("atlas_sim_alloc", int(nbytes), None, ctypes.byref(buffer))
        else:
            data = np.ascontiguousarray(np.frombuffer(init, np.uint8) if isinstance(init, bytes) else init)
            if data.nbytes != nbytes:
                raise ValueError("initial data size mismatch")
            self._call("atlas_sim_alloc", int(nbytes), data.ctypes.data_as(ctypes.c_void_p), ctypes.byref(buffer))
        self.sizes.append(int(nbytes))
        return buffer.value

    def upload(self, buffer: int, data: np.ndarray, offset: int = 0) -> None:
        data = np.ascontiguousarray(data)
        self._call("atlas_sim_upload", buffer, offset, data.ctypes.data_as(ctypes.c_void_p), data.nbytes)

    def read(self, buffer: int, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dtype = np.dtype(dtype)
        if count is None:
            count = (self.sizes[buffer] - offset) // dtype.itemsize
        out = np.empty(count, dtype)
        if count:
            self._call("atlas_sim_read", buffer, offset, out.ctypes.data_as(ctypes.c_void_p), out.nbytes)
        return out

    def zero(self, buffer: int, offset: int = 0, nbytes: int | None = None) -> None:
        if nbytes is None:
            nbytes = self.sizes[buffer] - offset
        self._call("atlas_sim_zero", buffer, offset, nbytes)

    def copy(self, dst: int, src: int, nbytes: int, dst_offset: int = 0, src_offset: int = 0) -> None:
        self._call("atlas_sim_copy", dst, dst_offset, src, src_offset, nbytes)

    def compile(self, source: str, kernels: list[str], options: list[str]) -> None:
        names = (ctypes.c_char_p * len(kernels))(*[k.encode() for k in kernels])
        opts = (ctypes.c_char_p * len(options))(*[o.encode() for o in options])
        self._call("atlas_sim_compile", source.encode(), names, len(kernels), opts, len(options))

    def set_schedule(self, launches: list[tuple[int, int, int, int]]) -> None:
        arr = (Launch * len(launches))(*[Launch(*l) for l in launches])
        self._call("atlas_sim_set_schedule", arr, len(launches))

    def set_epilogue(self, launches: list[tuple[int, int, int, int]]) -> None:
        """Launches run once after the last tick of every run, with that tick."""
        arr = (Launch * max(1, len(launches)))(*[Launch(*l) for l in launches])
        self._call("atlas_sim_set_epilogue", arr, len(launches))

    def set_persistent(self, launch: tuple[int, int, int, int] | None, barrier_buffer: int = 0,
                       ticks_per_launch: int = 0, plain: bool = False) -> None:
        """Cooperative launches of `launch` running up to ticks_per_launch ticks each, the buffer
        barrier_buffer zeroed before each (None: off); `plain`: ordinary launches whose residency
        the kernel's occupancy guarantees."""
        arr = Launch(*(launch or (0, 1, 1, 0)))
        self._call("atlas_sim_set_persistent", ctypes.byref(arr), barrier_buffer, ticks_per_launch if launch else 0,
                   PERSISTENT_PLAIN if plain else 0)

    def run(self, start_tick: int, ticks: int) -> RunStats:
        stats = RunStats()
        self._call("atlas_sim_run", start_tick, ticks, ctypes.byref(stats))
        return stats

    def fixed_indegree(self, spec: FixedIndegree) -> None:
        self._call("atlas_sim_fixed_indegree", ctypes.byref(spec))

    def build_slots(self, spec: "SlotTable") -> int:
        """Fill a counting group's slot table; returns the largest segment (the table is usable
        only when it is at most 15)."""
        largest = ctypes.c_uint32()
        self._call("atlas_sim_build_slots", ctypes.byref(spec), ctypes.byref(largest))
        return int(largest.value)

    def extract_spikes(self, buffer: int, rows: int, words: int, neurons: int) -> np.ndarray:
        count = ctypes.c_uint64()
        self._call("atlas_sim_extract_spikes", buffer, rows, words, neurons, None, 0, ctypes.byref(count))
        pairs = np.empty((count.value, 2), np.int64)
        if count.value:
            self._call("atlas_sim_extract_spikes", buffer, rows, words, neurons,
                       pairs.ctypes.data_as(ctypes.c_void_p), count.value, ctypes.byref(count))
        return pairs

    def set_profiling(self, enabled: bool) -> None:
        self._call("atlas_sim_set_profiling", 1 if enabled else 0)

    def kernel_time(self, kernel: int) -> tuple[float, int]:
        ms = ctypes.c_double()
        n = ctypes.c_uint64()
        self._call("atlas_sim_kernel_time", kernel, ctypes.byref(ms), ctypes.byref(n))
        return ms.value, n.value

    def device_name(self) -> str:
        """The device's marketing name and gcn architecture, read from its properties."""
        name = ctypes.create_string_buffer(512)
        self._call("atlas_sim_device_name", name, len(name))
        return name.value.decode(errors="replace")

    def close(self) -> None:
        if getattr(self, "_handle", None):
            self._lib.atlas_sim_destroy(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
