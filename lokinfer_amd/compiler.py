"""Compiling a function (the reference's lk.compile / lk.load / compile_ir, python/lokinfer/compiler.py:94-231 in
lariaus/lokinfer), two ways:

- `compile(fn, inputs=... | input_types=...)`: traces `fn` on symbolic values into the reference's text IR
  (lokinfer_amd.graph), runs the compiler passes in the C++ runtime and builds an executable: constants in one
  device arena, init run once, statically shaped calls captured into hipGraphs. The result saves to / loads from
  .lkm v2 files (`CompiledModel.save`, `load`).
- `capture(fn)`: runs `fn` eagerly once per input-shape signature, then captures it with torch's stream capture
  and replays that hipGraph. It keeps the concurrent branches a function opens on side streams (the Kokoro
  forward's), which the single-stream executable runs one after the other.
"""
from __future__ import annotations

import gc

import torch

from .graph import BufferType, ScalarType, TensorType, Value, Dim, Sym, tracing, Graph
from .runtime import GpuContext
from .tensor import Tensor, f32, from_numpy, i64


def _sig(args) -> tuple:
    return tuple((tuple(a.shape), a.dtype.name) for a in args)


class _Entry:
    def __init__(self, fn, args: list[Tensor], use_graph: bool, mutable: tuple = ()):
        ctx = GpuContext.shared()
        self.mutable = frozenset(mutable)
        # mutable inputs (written in place, e.g. a caller-owned KV cache) are bound by reference: the entry (and its
        # graph) uses the caller's buffer itself; the others are copied into the entry's own input buffers
        self.inputs = [a if i in self.mutable else Tensor(torch.empty_like(a.t, device=ctx.device))
                       for i, a in enumerate(args)]
        for i, (s, a) in enumerate(zip(self.inputs, args)):
            if i not in self.mutable:
                s.t.copy_(a.t)
        out = fn(*self.inputs)  # eager warm-up: binds shapes, builds lazy constants
        self.single = not isinstance(out, (tuple, list))
        self.graph = None
        self.fn = fn
        if use_graph:
            torch.cuda.synchronize()
            self.graph = torch.cuda.CUDAGraph()
            # No garbage collection while capturing: a collected model (models reference their compiled function
            # and back, so only the cycle collector frees them) destroys its own captured graphs and their memory
            # pools, which must not happen during a capture. Unreachable objects are collected before it instead.
            gc.collect()
            enabled = gc.isenabled()
            gc.disable()
            try:
                with torch.cuda.graph(self.graph):
                    out = fn(*self.inputs)
            finally:
                if enabled:
                    gc.enable()
        self.outputs = [out] if self.single else list(out)
        self.fresh = not use_graph  # eager: the warm-up already computed the first call's outputs

    def run(self, args):
        if self.fresh:
            self.fresh = False
            return self.outputs
        for i, (s, a) in enumerate(zip(self.inputs, args)):
            if i not in self.mutable:
                s.t.copy_(a.t, non_blocking=True)
        if self.graph is not None:
            self.graph.replay()
            outs = self.outputs
        else:
            out = self.fn(*self.inputs)
            outs = [out] if self.single else list(out)
        return outs


class CapturedModel:
    """A function replayed from torch stream capture, one graph per input-shape signature (see `capture`)."""

    MAX_ENTRIES = 16  # graphs kept per model (least recently used dropped first)

    def __init__(self, fn, use_graph: bool = True, mutable: tuple = (), by_ref: tuple = ()):
        self.fn = fn
        self.use_graph = use_graph
        self.mutable = tuple(sorted(set(mutable) | set(by_ref)))
        self._entries: dict[tuple, _Entry] = {}

    def _entry(self, args) -> _Entry:
        # an input bound by reference is part of the signature by address: the captured graph reads (or writes)
        # that buffer itself
        key = _sig(args) + tuple(args[i].t.data_ptr() for i in self.mutable)
        e = self._entries.pop(key, None)
        if e is None:
            if len(self._entries) >= self.MAX_ENTRIES:
                self._entries.pop(next(iter(self._entries)))
            e = _Entry(self.fn, list(args), self.use_graph, self.mutable)
        self._entries[key] = e  # most recently used last
        return e

    def run_inplace(self, *args):
        """Replays and returns the graph's own output tensors (overwritten by the next call)."""
        outs = self._entry(args).run(args)
        return outs[0] if len(outs) == 1 else tuple(outs)

    def __call__(self, *args):
        """Runs and returns fresh output tensors (copies of the graph's outputs)."""
        outs = self._entry(args).run(args)
        res = [Tensor(o.t.clone()) for o in outs]
        return res[0] if len(res) == 1 else tuple(res)


def capture(fn, inputs=None, graph: bool = True, mutable: tuple = (), by_ref: tuple = ()) -> CapturedModel:
    """Stream-captured `fn`: shapes are bound per call signature. `mutable`: indices of the inputs that the function
    writes in place (the reference's lk.MutableType inputs): bound by reference, one entry per buffer. `by_ref`:
    read-only inputs bound the same way, so that a call with the same buffers replays with no input copy (the
    other inputs are copied into the graph's own buffers on every call)."""
    m = CapturedModel(fn, use_graph=graph, mutable=mutable, by_ref=by_ref)
    if inputs is not None:
        m._entry(list(inputs))
    return m


# ---- traced compilation through the C++ runtime -----------------------------------------------------------------

class Pending:
    """Handle of an asynchronous call (`CompiledModel.submit`); `wait()` returns what the call returns."""

    __slots__ = ("_future",)

    def __init__(self, future):
        self._future = future

    def done(self) -> bool:
        return self._future.done()

    def wait(self, timeout: float | None = None):
        return self._future.result(timeout)


class CompiledModel:
    """A compiled model on the GPU (reference CompiledModel, python/lokinfer/compiler.py:94-184): `model(*inputs)`
    returns fresh output tensors, `run_inplace` the executable's own output buffers (overwritten by its next
    call); `save` writes a self-contained .lkm."""

    def __init__(self, exe, model, text: str, input_types: list, single: bool, externals: dict | None = None):
        self._exe = exe
        self._model = model
        self._externals = dict(externals or {})
        self.source_ir = text
        self.input_types = input_types
        self._single = single
        self._worker = None

    @property
    def uses_gpu(self) -> bool:
        return True

    def ir_text(self) -> str:
        """The IR after the compiler pipeline."""
        return self._model.text()

    @property
    def num_external_constants(self) -> int:
        return len(self._externals)

    def stats(self) -> dict:
        return self._exe.stats()

    def internalize(self) -> "CompiledModel":
        """Copies the captured tensors (external constants) into the model, so later writes to them no longer
        reach it (reference CompiledModel.internalize). The executable is re-created."""
        self._drain()
        if self._externals:
            from .rt import Executable

            self._model.internalize(self._externals)
            self._externals = {}
            self._exe = Executable(self._model, {})
        return self

    def save(self, path: str, *, bake_init: bool = False) -> None:
        """Writes a self-contained .lkm v2 (captured weights internalized). bake_init=True stores init's results
        (e.g. transposed weights) instead of their inputs, so loading does no init work (reference
        CompiledModel.save, compiler.py:112-117)."""
        self._drain()
        if bake_init:
            model, _ = self._model.bake_init(self._externals)
            model.internalize(self._externals)
            model.save(path)
            return
        if self._externals:
            self._model.internalize(self._externals)  # the executable keeps its bound device copies
            self._externals = {}
        self._model.save(path)

    def bake_init(self) -> dict:
        """Runs init once and replaces its computed results (weights transformed by hoisted kernels) with constants;
        init work nothing else needs is removed and the executable is re-created. Arenas, persistent state and
        models whose init defines symbols are left alone. Returns statistics (baked, baked_bytes,
        init_ops_before, init_ops_after) (reference CompiledModel.bake_init, compiler.py:119-127)."""
        from .rt import Executable

        self._drain()
        model, stats = self._model.bake_init(self._externals)
        self._exe = Executable(model, self._externals)
        self._model = model
        return stats

    def _call(self, args, copy: bool):
        outs = self._exe.run(list(args))
        if copy:
            outs = [Tensor(o.t.clone()) for o in outs]
        return outs[0] if self._single else tuple(outs)

    def __call__(self, *args):
        if self._worker is not None:
            return self.submit(*args).wait()
        return self._call(args, True)

    def run_inplace(self, *args):
        """Outputs over the executable's own memory, no copy (valid until the next call)."""
        return self._call(args, False)

    def submit(self, *args) -> Pending:
        """Runs the call on the model's worker thread (calls of one model run in submit order)."""
        if self._worker is None:
            from concurrent.futures import ThreadPoolExecutor

            self._worker = ThreadPoolExecutor(max_workers=1, thread_name_prefix="lokinfer-model")
        return Pending(self._worker.submit(self._call, args, True))

    def _drain(self):
        if self._worker is not None:
            self._worker.submit(lambda: None).result()


def _input_type(x, i: int, dynamic: bool):
    if isinstance(x, (TensorType, ScalarType)):
        return x
    if hasattr(x, "shape") and hasattr(x, "dtype") and not isinstance(x, Tensor):
        import numpy as np

        x = from_numpy(np.ascontiguousarray(x))
    if isinstance(x, Tensor):
        shape = [Sym(f"D{i}_{j}") for j in range(x.ndim)] if dynamic else list(x.shape)
        return TensorType(x.dtype, shape)
    if isinstance(x, float):
        return ScalarType(f32)
    if isinstance(x, int):
        return ScalarType(i64)
    raise TypeError(f"unsupported input {type(x).__name__}")


def compile(fn, inputs=None, *, dynamic: bool = False, input_types=None, pipeline=None,
            graphs: bool = True, lanes: int = 1) -> CompiledModel:
    """Traces `fn` on symbolic values and compiles it (reference lk.compile).

    inputs       example tensors / arrays / scalars (static shapes unless dynamic=True)
    dynamic      every input dim becomes its own symbol
    input_types  explicit TensorType / BufferType (mutable) / ScalarType list, e.g. [TensorType(f32, [Sym("N"), 4])]
    pipeline     the compiler passes (default: dce, bufferize, plan-memory, hoist-init)
    graphs       capture statically shaped calls into hipGraphs
    lanes        the most concurrent lanes of a statically shaped call's graph. A function that issues branches on side
                 streams (GpuContext.branch / join / mark / wait_mark) keeps that structure: each stream is a lane,
                 captured on a stream of its own with the function's waits plus the data dependencies. Otherwise
                 kernels are assigned to lanes from their data dependencies and the captured graph's edges follow
                 the lanes. Either way independent branches run concurrently on replay, and every call still
                 enqueues on torch's current stream
    """
    from .rt import Executable, Model

    if input_types is None:
        if inputs is None:
            raise ValueError("give inputs or input_types")
        input_types = [_input_type(x, i, dynamic) for i, x in enumerate(inputs)]
    g = Graph()
    args = [g.arg(t, f"in{i}_") for i, t in enumerate(input_types)]
    with tracing(g):
        out = fn(*args)
    single = isinstance(out, Value)
    outs = [out] if single else list(out)
    if not all(isinstance(o, Value) for o in outs):
        raise TypeError("the traced function must return traced values")
    text = g.to_text(outs)
    model = Model.parse(text).run_passes(pipeline if pipeline is not None else "pipeline")
    exe = Executable(model, g.externals, graphs=graphs, lanes=lanes)
    return CompiledModel(exe, model, text, input_types, single, g.externals)


def load(path: str, graphs: bool = True, lanes: int = 1) -> CompiledModel:
    """Loads a .lkm written by CompiledModel.save (or by the reference's writeModelFile): mmapped, constants
    uploaded once."""
    from .rt import Executable, Model

    model = Model.load(path)
    exe = Executable(model, {}, graphs=graphs, lanes=lanes)
    return CompiledModel(exe, model, model.text(), [], model.num_outputs == 1)


def compile_ir(text: str, *, externals: dict | None = None, internals: dict | None = None, pipeline=None,
               single: bool = True, graphs: bool = True) -> CompiledModel:
    """Compiles text IR directly: const.external data by name (lk.Tensors, bound by reference) and const.internal
    data by name (arrays, copied) (reference compile_ir)."""
    import numpy as np

    from .rt import Executable, Model

    model = Model.parse(text)
    for name, arr in (internals or {}).items():
        model.set_constant(name, np.ascontiguousarray(arr))
    model.run_passes(pipeline if pipeline is not None else "pipeline")
    ext = {k: (v if isinstance(v, Tensor) else from_numpy(np.ascontiguousarray(v))) for k, v in (externals or {}).items()}
    exe = Executable(model, ext, graphs=graphs)
    return CompiledModel(exe, model, text, [], single, ext)
