"""CPU-side checks of the C-ABI boundary: the library loads, exports every symbol include/lokinfer_hip.h
declares, and its registry holds every GPU kernel name the Python ops launch (reference
tests/python/test_registry.py:19-29 checks the same two-way agreement)."""
import re
from pathlib import Path

import lokinfer_amd as lk
from lokinfer_amd import _lib, ops

ROOT = Path(__file__).resolve().parent.parent


def header_symbols():
    text = (ROOT / "include" / "lokinfer_hip.h").read_text()
    return set(re.findall(r"\b(lk_\w+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    declared = header_symbols()
    assert len(declared) > 20
    L = _lib.lib()
    missing = [s for s in sorted(declared) if not hasattr(L, s)]
    assert not missing, missing


def test_registry_names_follow_the_device_convention():
    names = lk.registered_kernels()
    assert names == sorted(names) and len(names) == len(set(names))
    L = _lib.lib()
    for n in names:
        h = L.lk_find_kernel(n.encode())
        assert h
        assert L.lk_kernel_is_gpu(h) == (1 if "gpu" in n.split("_") else 0), n


def test_every_python_op_kernel_is_registered():
    src = (ROOT / "lokinfer_amd" / "ops.py").read_text()
    launched = set(re.findall(r'"(\w+_gpu(?:_mps)?)"', src))
    names = set(lk.registered_kernels())
    assert launched <= names, sorted(launched - names)


def test_unknown_kernel_and_bad_arity_are_errors():
    L = _lib.lib()
    assert not L.lk_find_kernel(b"no_such_kernel_f32_gpu")
    import ctypes as C

    h = L.lk_find_kernel(b"add_f32_gpu")
    rc = L.lk_run_kernel(h, (C.c_void_p * 1)(None), 1, (C.c_int64 * 1)(0), 0, (C.c_double * 1)(0), 0, None, 0, None)
    assert rc != 0 and b"wrong number of operands" in L.lk_last_error()


def test_ops_reject_cpu_operands():
    import pytest

    x = lk.zeros(2, 2)
    with pytest.raises(ops.OpError):
        ops.add_f32_gpu(x, x)
