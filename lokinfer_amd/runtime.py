"""HIP execution context: one stream (torch's current stream on the device), one zero-initialised device
workspace for kernels that merge partial results, and the launch path into the C-ABI registry.

Replaces the reference's GpuContext (src/runtime/gpu_internal.h:53-290): Metal command buffers, arg tables and
the params ring become plain HIP launches on one stream; errors come back as a status + message and are raised
as LokinferError, the binding-level exception the reference raises from Status (python/ext/module.cpp:29-31).
"""
from __future__ import annotations

import ctypes as C

import torch

from ._lib import LokinferError, check_device_errors, lib
from .graph import current_graph

WORKSPACE_BYTES = 64 << 20


class GpuContext:
    _shared: "GpuContext | None" = None

    def __init__(self):
        if not torch.cuda.is_available():
            raise LokinferError("no HIP device available (the lokinfer GPU kernels need an MI355X / gfx950)")
        self.device = torch.device("cuda", torch.cuda.current_device())
        # First 64 KiB: ticket counters (must start at zero; kernels restore them), rest: partials.
        self.workspace = torch.zeros(WORKSPACE_BYTES // 4, dtype=torch.float32, device=self.device)
        self.lib = lib()
        self._handles: dict[str, int] = {}
        self._ws_by_slot: dict[int, torch.Tensor] = {0: self.workspace}
        self.slot = 0

    def workspace_for(self, slot: int) -> torch.Tensor:
        """Workspace of a branch slot. Kernels on one stream are ordered and share slot 0; a branch that runs
        concurrently on another stream (see `branch`) uses its own slot. A new slot is allocated on first use,
        which happens on a model's eager warm-up run, before any graph capture."""
        ws = self._ws_by_slot.get(slot)
        if ws is None:
            if torch.cuda.is_current_stream_capturing():
                raise LokinferError("no workspace for this branch yet: run the function once outside capture")
            ws = torch.zeros(WORKSPACE_BYTES // 4, dtype=torch.float32, device=self.device)
            self._ws_by_slot[slot] = ws
        return ws

    def branch(self, stream: "torch.cuda.Stream", slot: int):
        """Context manager: run the enclosed launches on `stream` (which first waits for the current stream)
        with workspace slot `slot`. Join with `join(stream)` before consuming the branch's outputs."""
        ctx = self

        class _Branch:
            def __enter__(self):
                cur = torch.cuda.current_stream(ctx.device)
                stream.wait_stream(cur)
                g = current_graph()
                if g is not None:
                    g.stream_wait(stream, cur)
                self._prev = ctx.slot
                self._sc = torch.cuda.stream(stream)
                self._sc.__enter__()
                ctx.slot = slot
                return stream

            def __exit__(self, *exc):
                ctx.slot = self._prev
                self._sc.__exit__(*exc)
                return False

        return _Branch()

    def join(self, stream: "torch.cuda.Stream") -> None:
        cur = torch.cuda.current_stream(self.device)
        cur.wait_stream(stream)
        g = current_graph()
        if g is not None:
            g.stream_wait(cur, stream)

    def mark(self, stream: "torch.cuda.Stream"):
        """An event recorded on `stream` now; `wait_mark(other, m)` makes `other` wait for it. Traced functions
        record the same structure for the compiled runtime's lane schedule."""
        ev = torch.cuda.Event()
        ev.record(stream)
        g = current_graph()
        return (ev, g.mark(stream) if g is not None else None)

    def wait_mark(self, stream: "torch.cuda.Stream", m) -> None:
        stream.wait_event(m[0])
        g = current_graph()
        if g is not None and m[1] is not None:
            g.wait_mark(stream, m[1])

    @classmethod
    def shared(cls) -> "GpuContext":
        if cls._shared is None:
            cls._shared = GpuContext()
        return cls._shared

    def handle(self, name: str) -> int:
        h = self._handles.get(name)
        if h is None:
            h = self.lib.lk_find_kernel(name.encode())
            if not h:
                raise LokinferError(f"unknown kernel '{name}'")
            self._handles[name] = h
        return h

    def run(self, name: str, ptrs, ints, floats) -> None:
        L = self.lib
        n_p, n_i, n_f = len(ptrs), len(ints), len(floats)
        pa = (C.c_void_p * max(1, n_p))(*ptrs)
        ia = (C.c_int64 * max(1, n_i))(*ints)
        fa = (C.c_double * max(1, n_f))(*floats)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        ws = self.workspace_for(self.slot)
        rc = L.lk_run_kernel(self.handle(name), pa, n_p, ia, n_i, fa, n_f, ws.data_ptr(), ws.numel() * 4, stream)
        if rc != 0:
            raise LokinferError(L.lk_last_error().decode())


def synchronize() -> None:
    """Waits for the GPU and raises LokinferError for a data error a kernel recorded (check_device_errors)."""
    torch.cuda.synchronize()
    check_device_errors()
