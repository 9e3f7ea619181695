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
    launched = set(re.findall(r'_launch\(\s*f?"(\w+_gpu(?:_mps)?)"', src))
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


def test_device_error_messages_and_codes():
    """Every code include/lokinfer_hip.h declares has its own message in the library (no GPU call)."""
    text = (ROOT / "include" / "lokinfer_hip.h").read_text()
    codes = dict((n, int(v)) for n, v in re.findall(r"\b(LK_DEVERR_\w+)\s*=\s*(\d+)", text))
    assert sorted(codes.values()) == [1, 2, 3, 4, 5]
    L = _lib.lib()
    msgs = {c: L.lk_device_error_message(c).decode() for c in codes.values()}
    assert len(set(msgs.values())) == len(msgs) and all("unknown" not in m for m in msgs.values())
    assert L.lk_device_error_message(0).decode() == "no error"
    assert "unknown" in L.lk_device_error_message(99).decode()


def test_check_device_errors_raises_the_recorded_error(monkeypatch):
    """check_device_errors turns the record lk_take_device_error returns into LokinferError with the message and
    detail, and returns quietly for code 0 (the library is replaced by a stand-in that returns fixed records)."""
    import ctypes as C

    import pytest

    real = _lib.lib()

    class Fake:
        def __init__(self, code, detail):
            self.code, self.detail = code, detail

        def lk_take_device_error(self, p):
            C.cast(p, C.POINTER(C.c_int64))[0] = self.detail
            return self.code

        def lk_device_error_message(self, code):
            return real.lk_device_error_message(code)

    monkeypatch.setattr(_lib, "lib", lambda: Fake(0, 0))
    _lib.check_device_errors()
    monkeypatch.setattr(_lib, "lib", lambda: Fake(1, 77))
    with pytest.raises(_lib.LokinferError, match=r"device error 1: a persistent kernel.*timed out.*detail 77"):
        _lib.check_device_errors()
    monkeypatch.setattr(_lib, "lib", lambda: Fake(-1, 0))
    with pytest.raises(_lib.LokinferError, match="could not read"):
        _lib.check_device_errors()


def test_registry_rejects_bad_shapes_before_any_launch():
    """Shape checks run on the host before a launch (null device pointers, no GPU needed): a U whose point count
    does not match the kernel size, V rows that are not whole (residue, point) blocks, and a short ints array
    (read as zeros, never past its end)."""
    import ctypes as C

    L = _lib.lib()
    k = L.lk_find_kernel(b"wino_mm_lc_f32_gpu")
    nop, nout = C.c_int(), C.c_int()
    L.lk_kernel_arity(k, C.byref(nop), C.byref(nout))
    n = nop.value + nout.value
    ptrs = (C.c_void_p * n)()

    def run(ints):
        arr = (C.c_int64 * len(ints))(*ints)
        return L.lk_run_kernel(k, ptrs, n, arr, len(ints), None, 0, None, 0, None), L.lk_last_error().decode()

    # v [rows, Ci], u [A, Ci, Co], b [Co], tr [n], x [L, Ci], out [Lo, Co]; attrs dilation, groups, kernel, padding,
    # tile (K = 3, tile 4: A = 6)
    v_rows, ci, co, lo = 6 * 130, 64, 64, 500
    good = [v_rows, ci, 6, ci, co, co, 60, lo, ci, lo, co, 1, 1, 3, 1, 4]
    rc, msg = run([v_rows, ci, 7] + good[3:])
    assert rc == 1 and "point count" in msg
    rc, msg = run([v_rows + 1, ci] + good[2:])
    assert rc == 1 and "multiple of dilation" in msg
    rc, msg = run(good[:5])
    assert rc == 1 and "wino_mm" in msg


def test_decode_step_ops_reject_bad_shapes_before_any_launch():
    """The fused decode-step ops check their shapes (and K % 4, K <= 1024) on the host, before any launch."""
    import ctypes as C

    L = _lib.lib()

    def run(name, ints, floats=(1e-5,)):
        k = L.lk_find_kernel(name.encode())
        assert k, name
        nop, nout = C.c_int(), C.c_int()
        L.lk_kernel_arity(k, C.byref(nop), C.byref(nout))
        n = nop.value + nout.value
        ptrs = (C.c_void_p * n)()
        arr = (C.c_int64 * len(ints))(*ints)
        fl = (C.c_double * len(floats))(*floats)
        return L.lk_run_kernel(k, ptrs, n, arr, len(ints), fl, len(floats), None, 0, None), L.lk_last_error().decode()

    # lm_head_ln_argmax: part [S, K], bias [K], res [1, K], gamma [K], beta [K], table [V, K] -> logits [1, V], i64 [1]
    S, K, V = 12, 768, 100
    good = [S, K, K, 1, K, K, K, V, K, 1, V, 1]
    bad_table = [S, K, K, 1, K, K, K, V, K + 4, 1, V, 1]
    rc, msg = run("lm_head_ln_argmax_f32_gpu", bad_table)
    assert rc == 1 and "lm_head_ln_argmax" in msg
    rc, msg = run("lm_head_ln_argmax_f32_gpu", good[:6])
    assert rc == 1 and "lm_head_ln_argmax" in msg
    # gemv_partial_embed_ln: table [V, K], id [1], table2 [P, K], id2 [1], gamma, beta [K], w [K, N]
    #   -> part [slices(K), N], sum [1, K]
    N, P = 2304, 1024
    slices = 12
    good = [V, K, 1, P, K, 1, K, K, K, N, slices, N, 1, K]
    rc, msg = run("gemv_partial_embed_ln_f32_gpu", good[:9] + [N, slices + 1, N, 1, K])
    assert rc == 1 and "gemv_partial_embed_ln" in msg
    rc, msg = run("gemv_partial_embed_ln_f32_gpu", [V, K, 2] + good[3:])
    assert rc == 1 and "gemv_partial_embed_ln" in msg


def test_front_end_names():
    """The reference's lk.* names resolve (python/lokinfer/__init__.py in lariaus/lokinfer): the f16 family under
    lk.ops.f16_gpu, the state / mutability names, and a version string."""
    assert lk.ops.f16_gpu.gemm_f16_gpu is not None
    for name in ("persistent_buffer", "MutableType", "Pending", "dim_read", "compile", "load", "ceildiv"):
        assert hasattr(lk, name), name
    assert isinstance(lk.__version__, str)
