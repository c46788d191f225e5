"""The C ABI library loads and exports every entry point its header declares.

No compute call is made: loading the library and resolving symbols needs no GPU.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

from atlas_hip import native

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))
LIBRARIES = {"atlas_sim.h": native.LIBRARY, "atlas_train.h": native.PACKAGE_ROOT / "libatlas_train_hip.so"}


def _declared(header: Path) -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:int|void|uint64_t)\s+\**\s*(\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def built():
    import __graft_entry__
    for source, output, extra in __graft_entry__.LIBRARIES:
        if not output.exists():
            __graft_entry__._hipcc(source, output, extra)
    return native.LIBRARY


def test_every_header_has_a_library():
    assert {h.name for h in HEADERS} == set(LIBRARIES)


def test_library_exports_every_declared_symbol(built):
    header = ROOT / "include" / "atlas_sim.h"
    declared = _declared(header)
    assert len(declared) == len(native.EXPORTS) >= 17
    lib = ctypes.CDLL(str(built))
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing
    assert sorted(declared) == sorted(native.EXPORTS)
    dynsym = subprocess.run(["nm", "-D", "--defined-only", str(built)], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in dynsym.splitlines() if line.strip()}
    assert set(declared) <= exported


def test_training_library_exports_every_declared_symbol(built):
    declared = _declared(ROOT / "include" / "atlas_train.h")
    assert declared == ["b2_train_hip_v2", "b2_train_cuda_v2", "b2_train_math_v1", "b2_train_hip_v2_static",
                        "atlas_rsnn_create",
                        "atlas_rsnn_destroy", "atlas_rsnn_set_batch", "atlas_rsnn_step", "atlas_rsnn_profile",
                        "atlas_rsnn_read"]
    path = LIBRARIES["atlas_train.h"]
    lib = ctypes.CDLL(str(path))
    assert all(hasattr(lib, name) for name in declared)
    lib.b2_train_math_v1.restype = ctypes.c_uint64
    assert lib.b2_train_math_v1() == 1


def test_binding_sets_every_prototype(built):
    lib = native.library()
    for name in native.EXPORTS:
        fn = getattr(lib, name)
        assert fn.argtypes, name


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(native, "_lib", None)
    monkeypatch.setattr(native, "LIBRARY", tmp_path / "absent.so")
    with pytest.raises(native.NativeUnavailable):
        native.library()


def test_oracle_library_is_separate_from_the_product(built):
    """The product library never links the CPU oracle."""
    needed = subprocess.run(["readelf", "-d", str(built)], capture_output=True, text=True).stdout
    assert "oracle" not in needed
    for path in (ROOT / "brian2-atlas_amd").rglob("*.py"):
        assert "import oracle" not in path.read_text() and "from oracle" not in path.read_text(), path


def test_recurrent_trainer_rejects_bad_specs_before_touching_a_gpu(built):
    """Spec validation happens on the host, before any HIP call."""
    from atlas_hip import rsnn
    lib = rsnn._library()
    plan = rsnn.recurrent_plan(batch=16, time=4, inputs=8, hidden=16, classes=3)
    w = [np.zeros(s, np.float32) for s in ((8, 16), (16, 16), (16, 3))]
    for bad in ({"hidden": 20}, {"batch": 0}, {"classes": 0}):
        spec = rsnn._Spec(*({**plan, **bad}[k] for k in ("batch", "time", "inputs", "hidden", "classes", "alpha",
                                                          "beta", "threshold", "slope", "learning_rate", "beta1",
                                                          "beta2", "epsilon")))
        handle = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(256)
        rc = lib.atlas_rsnn_create(ctypes.byref(spec), *(rsnn._ptr(a) for a in w), ctypes.byref(handle), buf, 256)
        assert rc == 7 and b"multiples of 16" in buf.value and not handle.value
