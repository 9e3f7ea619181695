"""Tracing: `lk.compile` runs a function on symbolic values and records every op as the reference's text IR
(docs/impl-notes/design-ir.md §5-7, python/lokinfer/graph.py in lariaus/lokinfer writes the same text). The text
is handed to the runtime (lokinfer_amd.rt), which parses it, runs the compiler passes and builds an executable.

  Dim          a symbolic dimension expression (Sym("T"), 600 * F, ...), kept in the runtime's canonical form
  TensorType   tensor<dtype[shape]> of an input; BufferType marks a mutable input (written in place)
  Value        a traced value: shape (ints and Dims), dtype
  Graph        the IR being recorded; `tracing(graph)` makes it current for the ops
"""
from __future__ import annotations

import contextlib
import re
import threading

import torch

from .tensor import DType, Tensor

_INT = re.compile(r"-?\d+")


class Dim:
    """A symbolic dim. Arithmetic with ints and Dims yields the runtime's canonical form (an int when constant).
    Equality is structural; ordering comparisons that cannot be decided at trace time are taken as true (the
    kernels and the runtime check the values per call)."""

    __slots__ = ("text",)

    def __init__(self, text: str):
        self.text = text

    @staticmethod
    def make(text: str):
        from .rt import dim_canonical

        c = dim_canonical(text)
        return int(c) if _INT.fullmatch(c) else Dim(c)

    def __str__(self):
        return self.text

    def __repr__(self):
        return f"Dim({self.text})"

    def __hash__(self):
        return hash(self.text)

    def __eq__(self, o):
        return isinstance(o, Dim) and o.text == self.text

    def __ne__(self, o):
        return not self.__eq__(o)

    def _bin(self, o, op, rev=False):
        if not isinstance(o, (int, Dim)):
            return NotImplemented
        a, b = (o, self) if rev else (self, o)
        return Dim.make(f"({a}) {op} ({b})")

    def __add__(self, o):
        return self._bin(o, "+")

    def __radd__(self, o):
        return self._bin(o, "+", True)

    def __sub__(self, o):
        return self._bin(o, "-")

    def __rsub__(self, o):
        return self._bin(o, "-", True)

    def __mul__(self, o):
        return self._bin(o, "*")

    def __rmul__(self, o):
        return self._bin(o, "*", True)

    def __floordiv__(self, o):
        return self._bin(o, "//")

    def __rfloordiv__(self, o):
        return self._bin(o, "//", True)

    def __mod__(self, o):
        return self._bin(o, "%")

    def __rmod__(self, o):
        return self._bin(o, "%", True)

    def __neg__(self):
        return Dim.make(f"-({self})")

    def __pos__(self):
        return self

    def _order(self, o):
        return True  # undecidable at trace time

    __lt__ = __le__ = __gt__ = __ge__ = _order

    def __int__(self):
        raise TypeError(f"symbolic dim {self.text} has no value at trace time")

    __index__ = __int__


def Sym(name: str) -> Dim:
    """A named symbol (reference lk.Sym)."""
    return Dim(name)


def ceildiv(a, b):
    if isinstance(a, int) and isinstance(b, int):
        return -(-a // b)
    return Dim.make(f"ceildiv({a}, {b})")


def dim_text(d) -> str:
    return str(d)


class TensorType:
    """tensor<dtype[shape]> (reference lk.TensorType)."""

    kind = "tensor"

    def __init__(self, dtype: DType, shape):
        self.dtype = dtype
        self.shape = tuple(d if isinstance(d, Dim) else int(d) for d in shape)

    def ir(self) -> str:
        return f"{self.kind}<{self.dtype.name}[{', '.join(dim_text(d) for d in self.shape)}]>"

    def __repr__(self):
        return self.ir()


class BufferType(TensorType):
    """A mutable input (reference lk.MutableType / buffer-typed input): the caller's buffer, written in place by
    `inout` kernels, bound without a copy."""

    kind = "buffer"


class ScalarType:
    """A host scalar input (reference lk.ScalarType)."""

    def __init__(self, dtype: DType):
        self.dtype = dtype
        self.shape = ()

    def ir(self) -> str:
        return self.dtype.name


class Value:
    """A value while tracing: the same shape / dtype surface as lk.Tensor, so the ops' shape rules run on it."""

    __slots__ = ("graph", "name", "type")

    def __init__(self, graph: "Graph", name: str, type_):
        self.graph = graph
        self.name = name
        self.type = type_

    @property
    def shape(self) -> tuple:
        return self.type.shape

    @property
    def dtype(self) -> DType:
        return self.type.dtype

    @property
    def ndim(self) -> int:
        return len(self.type.shape)

    @property
    def device(self) -> str:
        return "gpu"

    def numel(self):
        n = 1
        for d in self.shape:
            n = n * d
        return n

    def __repr__(self) -> str:
        return f"%{self.name}: {self.type.ir()}"


def _attr_text(v) -> str:
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, int):
        return str(v)
    if isinstance(v, float):
        r = repr(v)
        return r if any(c in r for c in ".einf") else r + ".0"
    if isinstance(v, str):
        return '"' + v.replace("\\", "\\\\").replace('"', '\\"') + '"'
    if isinstance(v, Dim):
        return f"dim<{v}>"
    if isinstance(v, (list, tuple)):
        if any(isinstance(x, float) for x in v):
            return "f[" + ", ".join(_attr_text(float(x)) for x in v) + "]"
        return "[" + ", ".join(str(int(x)) for x in v) + "]"
    raise TypeError(f"unsupported attribute value {v!r}")


class Graph:
    """The IR recorded while tracing one function."""

    def __init__(self):
        self.args: list[Value] = []
        self.lines: list[str] = []
        self.externals: dict[str, Tensor] = {}  # const.external name -> the captured tensor
        self._ext_of: dict[int, tuple] = {}      # id(tensor) -> (tensor, value)
        self._n = 0
        # stream structure of the traced function (GpuContext.branch / join / wait): lane 0 is the stream tracing
        # began on, other streams get lanes 1, 2, ... in first-use order; every kernel has a trace sequence number,
        # and a stream's wait on another is kept as (lane, last sequence number issued there) for the next kernel
        # the waiting stream issues
        self.base_stream = None
        self._lanes: dict[int, int] = {}
        self._seq = 0
        self._last_seq: dict[int, int] = {}       # lane -> sequence number of its last kernel
        self._pending: dict[int, list] = {}       # lane -> [(lane, seq)] for its next kernel
        self._kernels: list[list] = []           # [line index, lane, seq, after]

    def _fresh(self, hint: str) -> str:
        self._n += 1
        return f"{hint}{self._n}"

    def fresh_symbol(self, hint: str) -> str:
        """A symbol name no dim of this graph uses yet."""
        return self._fresh(hint)

    def arg(self, type_, hint: str = "in") -> Value:
        v = Value(self, self._fresh(hint), type_)
        self.args.append(v)
        return v

    def value_of(self, x) -> Value:
        """A traced value for an op operand: a Value of this graph, or a concrete lk.Tensor captured as a
        const.external (bound by reference when the executable is created)."""
        if isinstance(x, Value):
            if x.graph is not self:
                raise ValueError("value belongs to another graph")
            return x
        if isinstance(x, Tensor):
            hit = self._ext_of.get(id(x))
            if hit is not None and hit[0] is x:
                return hit[1]
            name = f"ext{len(self.externals)}"
            t = TensorType(x.dtype, x.shape)
            v = Value(self, self._fresh("c"), t)
            self.lines.append(f'%{v.name} = const.external @"{name}" {{device = "{x.device}"}} : {t.ir()}')
            self.externals[name] = x
            self._ext_of[id(x)] = (x, v)
            return v
        raise TypeError(f"expected a traced value or lk.Tensor, got {type(x).__name__}")

    def lane_of(self, stream) -> int:
        h = stream.cuda_stream
        if self.base_stream is None or h == self.base_stream:
            return 0
        return self._lanes.setdefault(h, len(self._lanes) + 1)

    def stream_wait(self, waiter, producer) -> None:
        """`waiter` waits for the kernels issued on `producer` so far (a fork, a join or an event)."""
        a, b = self.lane_of(waiter), self.lane_of(producer)
        if a != b and b in self._last_seq:
            self._pending.setdefault(a, []).append((b, self._last_seq[b]))

    def mark(self, stream) -> tuple:
        """An event recorded on `stream`: what a later wait_mark waits for."""
        b = self.lane_of(stream)
        return (b, self._last_seq.get(b, -1))

    def wait_mark(self, waiter, mark: tuple) -> None:
        a = self.lane_of(waiter)
        if mark[0] != a and mark[1] >= 0:
            self._pending.setdefault(a, []).append(mark)

    def kernel(self, name: str, operands: list, attrs: dict, result_types: list) -> list[Value]:
        lane = self.lane_of(torch.cuda.current_stream()) if self.base_stream is not None else 0
        vals = [self.value_of(x) for x in operands]
        results = [Value(self, self._fresh("v"), t) for t in result_types]
        self._kernels.append([len(self.lines), lane, self._seq, self._pending.pop(lane, []),
                              (name, vals, dict(attrs), results, result_types)])
        self._last_seq[lane] = self._seq
        self._seq += 1
        self.lines.append(self._kernel_line(name, vals, attrs, results, result_types))
        return results

    @staticmethod
    def _kernel_line(name, vals, attrs, results, result_types) -> str:
        attr = ""
        if attrs:
            attr = " {" + ", ".join(f"{k} = {_attr_text(attrs[k])}" for k in sorted(attrs)) + "}"
        lhs = ", ".join(f"%{r.name}" for r in results)
        types = ", ".join(t.ir() for t in result_types)
        ops = ", ".join(f"%{v.name}" for v in vals)
        return (f"{lhs} = " if results else "") + f'kernel "{name}"({ops}){attr}' + (f" : {types}" if results else "")

    def view(self, x, type_, offset=0) -> Value:
        src = self.value_of(x)
        v = Value(self, self._fresh("v"), type_)
        self.lines.append(f"%{v.name} = view %{src.name}[{offset}] : {type_.ir()}")
        return v

    def sync(self, x, kind: str) -> Value:
        src = self.value_of(x)
        v = Value(self, self._fresh("s"), src.type)
        self.lines.append(f"%{v.name} = sync {kind} %{src.name} : {src.type.ir()}")
        return v

    def persistent(self, type_, device: str = "gpu") -> Value:
        """Model-lifetime state (buffer.alloc {persistent}), written in place by `inout` kernels."""
        bt = BufferType(type_.dtype, type_.shape)
        v = Value(self, self._fresh("p"), bt)
        self.lines.append(f'%{v.name} = buffer.alloc {{device = "{device}", persistent = true}} : {bt.ir()}')
        return v

    def dim_read(self, x, index: int, symbol: str) -> Dim:
        src = self.value_of(x)
        self.lines.append(f"dim.read %{src.name}[{int(index)}] -> {symbol}")
        return Dim(symbol)

    def _stream_attrs(self) -> None:
        """Once any kernel ran on a side stream, every kernel line carries its lane, sequence number and waits as
        string attributes (no kernel argument: the executable's lane schedule reads them)."""
        if not any(k[1] for k in self._kernels):
            return
        for idx, lane, seq, after, (name, vals, attrs, results, types) in self._kernels:
            extra = dict(attrs, lane=str(lane), seq=str(seq))
            if after:
                extra["after"] = ",".join(f"{l}:{q}" for l, q in after)
            self.lines[idx] = self._kernel_line(name, vals, extra, results, types)

    def to_text(self, outputs: list[Value]) -> str:
        self._stream_attrs()
        args = ", ".join(f"%{a.name}: {a.type.ir()}" + (" mutable" if isinstance(a.type, BufferType) else "")
                         for a in self.args)
        types = [o.type.ir() for o in outputs]
        res = f" -> {types[0]}" if len(types) == 1 else f" -> ({', '.join(types)})"
        body = "".join(f"    {line}\n" for line in self.lines)
        ret = ", ".join(f"%{o.name}" for o in outputs)
        return f"model {{\n  init {{\n    return\n  }}\n  exec({args}){res} {{\n{body}    return {ret}\n  }}\n}}\n"


_state = threading.local()


def current_graph() -> Graph | None:
    return getattr(_state, "graph", None)


@contextlib.contextmanager
def tracing(graph: Graph):
    prev = current_graph()
    if graph.base_stream is None and torch.cuda.is_available():
        graph.base_stream = torch.cuda.current_stream().cuda_stream
    _state.graph = graph
    try:
        yield graph
    finally:
        _state.graph = prev
