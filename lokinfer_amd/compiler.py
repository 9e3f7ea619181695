"""`lk.compile`: turns a function of tensors into a replayable HIP graph per input-shape signature.

The reference traces the function into text IR and runs a 4-pass compiler plus an instruction interpreter
(python/lokinfer/compiler.py:94-231, src/runtime/executable.cpp:567-1144 in lariaus/lokinfer). On MI355X the
equivalent of "compile once, run many" is stream capture: the first call with a new shape signature runs the
function eagerly (binding the symbolic sizes, uploading captured constants, warming the kernels), then runs it
again under hipStreamBeginCapture; later calls copy the inputs into the captured input buffers and replay the
hipGraph (one launch for the whole forward, no per-kernel host work). All intermediates live in the graph's
private memory pool, which plays the role of the reference's planned arena (plan-memory pass).

Functions must be capturable: GPU work only between inputs and outputs (no host reads of device data).
"""
from __future__ import annotations

import gc

import torch

from .runtime import GpuContext
from .tensor import Tensor


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


class CompiledModel:
    """Callable compiled function (reference CompiledModel, python/lokinfer/compiler.py:94-184)."""

    def __init__(self, fn, use_graph: bool = True, mutable: tuple = ()):
        self.fn = fn
        self.use_graph = use_graph
        self.mutable = tuple(mutable)
        self._entries: dict[tuple, _Entry] = {}

    def _entry(self, args) -> _Entry:
        # a mutable input is part of the signature by address: the captured graph writes that buffer
        key = _sig(args) + tuple(args[i].t.data_ptr() for i in self.mutable)
        e = self._entries.get(key)
        if e is None:
            e = _Entry(self.fn, list(args), self.use_graph, self.mutable)
            self._entries[key] = e
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


def compile(fn, inputs=None, input_types=None, graph: bool = True, mutable: tuple = ()) -> CompiledModel:
    """Compiles `fn` (reference lk.compile, python/lokinfer/compiler.py:187-212). `inputs` / `input_types` are
    accepted for API compatibility; shapes are bound per call signature. `mutable`: indices of the inputs that the
    function writes in place (the reference's lk.MutableType inputs): bound by reference, one entry per buffer."""
    m = CompiledModel(fn, use_graph=graph, mutable=mutable)
    if inputs is not None:
        m._entry(list(inputs))
    return m
