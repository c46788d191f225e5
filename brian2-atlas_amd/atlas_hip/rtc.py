"""Device-free hiprtc compilation of a generated tick module (gfx950 code object).

Used by ``__graft_entry__.build()`` and the CPU test suite to prove that the
hand-written templates plus the generated statement bodies compile for gfx950
without a GPU.  The runtime library performs the same compilation on the device
host before loading the module.
"""
from __future__ import annotations

import ctypes
import ctypes.util
from pathlib import Path

_CANDIDATES = ["/opt/rocm/lib/libhiprtc.so", "libhiprtc.so"]


def _library() -> ctypes.CDLL:
    for name in _CANDIDATES:
        try:
            return ctypes.CDLL(name)
        except OSError:
            continue
    found = ctypes.util.find_library("hiprtc")
    if found:
        return ctypes.CDLL(found)
    raise OSError("libhiprtc.so not found")


class CompileError(RuntimeError):
    pass


def compile_source(source: str, options: list[str]) -> bytes:
    """Return the gfx950 code object for ``source``; raise CompileError with the log."""
    lib = _library()
    prog = ctypes.c_void_p()
    rc = lib.hiprtcCreateProgram(ctypes.byref(prog), source.encode(), b"atlas_model.hip", 0, None, None)
    if rc != 0:
        raise CompileError(f"hiprtcCreateProgram failed ({rc})")
    opts = (ctypes.c_char_p * len(options))(*[o.encode() for o in options])
    rc = lib.hiprtcCompileProgram(prog, len(options), opts)
    size = ctypes.c_size_t()
    lib.hiprtcGetProgramLogSize(prog, ctypes.byref(size))
    log = ctypes.create_string_buffer(size.value + 1)
    lib.hiprtcGetProgramLog(prog, log)
    if rc != 0:
        lib.hiprtcDestroyProgram(ctypes.byref(prog))
        raise CompileError(log.value.decode(errors="replace"))
    lib.hiprtcGetCodeSize(prog, ctypes.byref(size))
    code = ctypes.create_string_buffer(size.value)
    lib.hiprtcGetCode(prog, code)
    lib.hiprtcDestroyProgram(ctypes.byref(prog))
    return code.raw


def compile_plan(plan) -> bytes:
    from . import engine
    return compile_source(plan.source, engine.COMPILE_OPTIONS)


def header_path() -> Path:
    from . import native
    return native.DEVICE_HEADER
