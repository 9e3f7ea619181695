"""ctypes binding of the compiled-model runtime (include/lokinfer_rt.h): models in the reference's text IR and .lkm
v2 format, the compiler passes, and executables that run a model on the GPU from one device arena.

It plays the part of the reference's nanobind module (python/ext/module.cpp in lariaus/lokinfer: compile_text,
load_model, save_model, create_executable, Executable.run). Device memory for inputs and outputs is torch's on
the Python side (plumbing only); every kernel runs through the HIP library.
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import LokinferError, lib
from .tensor import DType, Tensor, f16, f32, i32, i64, u8

# the .lkm dtype codes (f32 0, f16 1, bf16 2, i8 3, u8 4, i16 5, i32 6, i64 7, bool 8)
_CODE = {"f32": 0, "f16": 1, "u8": 4, "i32": 6, "i64": 7}
_BY_CODE = {0: f32, 1: f16, 4: u8, 6: i32, 7: i64}


class LkTensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("shape", C.c_int64 * 8), ("rank", C.c_int32), ("dtype", C.c_int32)]


_bound = False


def _rt():
    global _bound
    L = lib()
    if _bound:
        return L
    vp, cp, i32_, u64 = C.c_void_p, C.c_char_p, C.c_int, C.c_uint64
    sig = {
        "lk_free": ([vp], None),
        "lk_model_parse": ([cp], vp),
        "lk_model_load": ([cp], vp),
        "lk_model_from_bytes": ([vp, u64], vp),
        "lk_model_save": ([vp, cp], i32_),
        "lk_model_to_bytes": ([vp, C.POINTER(vp), C.POINTER(u64)], i32_),
        "lk_model_print": ([vp], vp),
        "lk_model_verify": ([vp], i32_),
        "lk_model_run_passes": ([vp, cp], i32_),
        "lk_model_set_constant": ([vp, cp, vp, u64, i32_], i32_),
        "lk_model_internalize": ([vp, i32_, C.POINTER(cp), C.POINTER(vp), C.POINTER(u64)], i32_),
        "lk_model_num_inputs": ([vp], i32_),
        "lk_model_num_outputs": ([vp], i32_),
        "lk_model_input_is_mutable": ([vp, i32_], i32_),
        "lk_model_bake_init": ([vp, i32_, C.POINTER(cp), C.POINTER(vp), C.POINTER(u64), C.POINTER(i32_), vp,
                                C.POINTER(u64)], vp),
        "lk_model_free": ([vp], None),
        "lk_dim_canonical": ([cp], vp),
        "lk_exe_create": ([vp, i32_, C.POINTER(cp), C.POINTER(vp), C.POINTER(u64), C.POINTER(i32_), vp, i32_], vp),
        "lk_exe_run": ([vp, i32_, C.POINTER(LkTensor), i32_, C.POINTER(LkTensor), C.POINTER(i32_), vp, i32_], i32_),
        "lk_exe_stats": ([vp, C.POINTER(u64), C.POINTER(u64), C.POINTER(i32_), C.POINTER(i32_)], i32_),
        "lk_exe_free": ([vp], None),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _bound = True
    return L


def _check(rc: int) -> None:
    if rc != 0:
        raise LokinferError(lib().lk_last_error().decode())


def dim_canonical(text: str) -> str:
    """The runtime's canonical form of a dim expression (the C++ DimPool's printing)."""
    L = _rt()
    p = L.lk_dim_canonical(text.encode())
    if not p:
        raise LokinferError(L.lk_last_error().decode())
    try:
        return C.string_at(p).decode()
    finally:
        L.lk_free(p)


class Model:
    """A model in the runtime's IR (reference lk::Model): parsed from text, loaded from a .lkm, transformed by the
    compiler passes, printed or saved."""

    def __init__(self, handle):
        if not handle:
            raise LokinferError(lib().lk_last_error().decode())
        self._h = handle
        self._keep: list = []  # host bytes the model's constants point to

    @classmethod
    def parse(cls, text: str) -> "Model":
        return cls(_rt().lk_model_parse(text.encode()))

    @classmethod
    def load(cls, path: str) -> "Model":
        return cls(_rt().lk_model_load(str(path).encode()))

    @classmethod
    def from_bytes(cls, data: bytes) -> "Model":
        buf = C.create_string_buffer(bytes(data), len(data))
        return cls(_rt().lk_model_from_bytes(C.cast(buf, C.c_void_p), len(data)))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _rt().lk_model_free(h)
            except Exception:  # interpreter shutdown: the library may already be gone
                pass
            self._h = None

    def text(self) -> str:
        L = _rt()
        p = L.lk_model_print(self._h)
        try:
            return C.string_at(p).decode()
        finally:
            L.lk_free(p)

    def to_bytes(self) -> bytes:
        L = _rt()
        p, n = C.c_void_p(), C.c_uint64()
        _check(L.lk_model_to_bytes(self._h, C.byref(p), C.byref(n)))
        try:
            return C.string_at(p, n.value)
        finally:
            L.lk_free(p)

    def save(self, path: str) -> None:
        _check(_rt().lk_model_save(self._h, str(path).encode()))

    def verify(self) -> None:
        _check(_rt().lk_model_verify(self._h))

    def run_passes(self, passes) -> "Model":
        names = passes if isinstance(passes, str) else ",".join(passes)
        _check(_rt().lk_model_run_passes(self._h, names.encode()))
        return self

    def set_constant(self, name: str, data) -> None:
        """The bytes of internal constant `name` (a numpy array or bytes; the model keeps a copy)."""
        b = bytes(memoryview(data).cast("B")) if not isinstance(data, bytes) else data
        _check(_rt().lk_model_set_constant(self._h, name.encode(), C.c_char_p(b), len(b), 1))

    def internalize(self, externals: dict) -> None:
        """const.external -> const.internal with copies of the given tensors' bytes (reference internalize)."""
        if not externals:
            return
        names = list(externals)
        data = [_host_bytes(externals[n]) for n in names]
        arr_n = (C.c_char_p * len(names))(*[n.encode() for n in names])
        arr_p = (C.c_void_p * len(names))(*[C.cast(C.c_char_p(d), C.c_void_p) for d in data])
        arr_s = (C.c_uint64 * len(names))(*[len(d) for d in data])
        _check(_rt().lk_model_internalize(self._h, len(names), arr_n, arr_p, arr_s))

    def bake_init(self, externals: dict | None = None) -> tuple["Model", dict]:
        """Runs init once (externals bound by name, as for an Executable) and returns (a new model whose computed
        init results are const.internal data, statistics) (reference rt::bakeInit)."""
        L = _rt()
        arrs, _keep = _ext_arrays(externals or {})
        st = (C.c_uint64 * 4)()
        h = L.lk_model_bake_init(self._h, *arrs, _stream(), st)
        if not h:
            raise LokinferError(L.lk_last_error().decode())
        return Model(h), {"baked": st[0], "baked_bytes": st[1], "init_ops_before": st[2], "init_ops_after": st[3]}

    @property
    def num_inputs(self) -> int:
        return _rt().lk_model_num_inputs(self._h)

    @property
    def num_outputs(self) -> int:
        return _rt().lk_model_num_outputs(self._h)

    def input_is_mutable(self, i: int) -> bool:
        return bool(_rt().lk_model_input_is_mutable(self._h, i))


def _host_bytes(x) -> bytes:
    t = x.t if isinstance(x, Tensor) else x
    if isinstance(t, torch.Tensor):
        return t.detach().contiguous().cpu().numpy().tobytes()
    return bytes(memoryview(t).cast("B"))


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ext_arrays(externals: dict):
    """(n, names, pointers, sizes, on_device) C arrays for externals bound by name, and the tensors to keep alive."""
    names = list(externals)
    ts = [externals[n] if isinstance(externals[n], Tensor) else Tensor(externals[n]) for n in names]
    n = len(names)
    arr_n = (C.c_char_p * max(n, 1))(*[x.encode() for x in names])
    arr_p = (C.c_void_p * max(n, 1))(*[t.data_ptr() for t in ts])
    arr_s = (C.c_uint64 * max(n, 1))(*[t.nbytes for t in ts])
    arr_d = (C.c_int * max(n, 1))(*[1 if t.device == "gpu" else 0 for t in ts])
    return (n, arr_n, arr_p, arr_s, arr_d), ts


class Executable:
    """A model loaded onto the GPU (reference lk::rt::Executable): constants uploaded once into one device arena,
    init run, calls replayed from captured hipGraphs for statically shaped calls. `externals` maps
    const.external names to lk.Tensors bound by reference (device) or uploaded (host)."""

    def __init__(self, model: Model, externals: dict | None = None, graphs: bool = True, lanes: int = 1):
        L = _rt()
        externals = externals or {}
        self.model = model
        self._ext = dict(externals)  # keeps the bound tensors alive
        arrs, self._ts = _ext_arrays(externals)
        flags = (1 if graphs else 0) | (max(1, min(int(lanes), 8)) << 8)
        self._h = L.lk_exe_create(model._h, *arrs, _stream(), flags)
        if not self._h:
            raise LokinferError(L.lk_last_error().decode())

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                torch.cuda.synchronize()
                _rt().lk_exe_free(h)
            except Exception:  # interpreter shutdown
                pass
            self._h = None

    def run(self, inputs: list, sync: bool = False) -> list[Tensor]:
        """One call on torch's current stream. Returns the outputs as tensors over the executable's own memory
        (overwritten by its next call)."""
        L = _rt()
        arr = (LkTensor * max(len(inputs), 1))()
        keep = []
        for i, x in enumerate(inputs):
            if isinstance(x, (int, float)):
                slot = C.c_int64(x) if isinstance(x, int) else C.c_double(x)
                keep.append(slot)
                arr[i].data = C.cast(C.pointer(slot), C.c_void_p)
                arr[i].rank = 0
                arr[i].dtype = 7 if isinstance(x, int) else 0
                continue
            t = x if isinstance(x, Tensor) else Tensor(x)
            if t.device != "gpu":
                t = Tensor(t.t.cuda())
                keep.append(t)
            arr[i].data = t.data_ptr()
            arr[i].rank = t.ndim
            arr[i].dtype = _CODE[t.dtype.name]
            for j, d in enumerate(t.shape):
                arr[i].shape[j] = d
        outs = (LkTensor * 16)()
        n_out = C.c_int(0)
        _check(L.lk_exe_run(self._h, len(inputs), arr, 16, outs, C.byref(n_out), _stream(), 1 if sync else 0))
        return [_wrap_out(outs[k], self) for k in range(n_out.value)]

    def stats(self) -> dict:
        m, c, g, s = C.c_uint64(), C.c_uint64(), C.c_int(), C.c_int()
        _check(_rt().lk_exe_stats(self._h, C.byref(m), C.byref(c), C.byref(g), C.byref(s)))
        return {"model_arena_bytes": m.value, "call_arena_bytes": c.value, "graphs": g.value, "lanes": s.value}


def _wrap_out(o: LkTensor, owner) -> Tensor:
    """A torch tensor over executable-owned device memory (no copy). The tensor keeps `owner` (the executable)
    alive, so its memory outlives every view; the values are overwritten by the executable's next call."""
    dt: DType = _BY_CODE[o.dtype]
    shape = [o.shape[j] for j in range(o.rank)]
    n = 1
    for d in shape:
        n *= d
    if n == 0:
        return Tensor(torch.empty(shape, dtype=dt.torch, device="cuda"))
    # wrap the raw device pointer through the CUDA array interface (torch-ROCm maps it to HIP)
    holder = _DevPtr(o.data, shape, dt, owner)
    return Tensor(torch.as_tensor(holder, device="cuda"))


class _DevPtr:
    """__cuda_array_interface__ over a device pointer the executable owns."""

    _TYPESTR = {"f32": "<f4", "f16": "<f2", "i64": "<i8", "i32": "<i4", "u8": "|u1"}

    def __init__(self, ptr: int, shape, dt: DType, owner=None):
        self.owner = owner
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": self._TYPESTR[dt.name],
                                         "data": (ptr, False), "version": 3, "strides": None}
