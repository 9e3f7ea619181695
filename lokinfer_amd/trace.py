"""Launch recording hooks used by `lk.compile` (compiler.py): while a recorder is active every kernel launch
and host->device copy is appended to it. Outside compilation these are no-ops."""
from __future__ import annotations

_active: list = []


def record(name, operands, outs, ints, floats) -> None:
    if _active:
        _active[-1].on_kernel(name, operands, outs, ints, floats)


def record_copy(src, dst) -> None:
    if _active:
        _active[-1].on_copy(src, dst)


class recording:
    def __init__(self, rec):
        self.rec = rec

    def __enter__(self):
        _active.append(self.rec)
        return self.rec

    def __exit__(self, *exc):
        _active.pop()
        return False
