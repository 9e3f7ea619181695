"""lokinfer_amd: an MI355X-native (CDNA4, gfx950) GPU backend with the lokinfer operator API.

`import lokinfer_amd as lk` gives the reference's front-end names (python/lokinfer/__init__.py in
lariaus/lokinfer): lk.Tensor, lk.from_numpy, lk.randn, lk.f32 / lk.i64, lk.ops.*_gpu, lk.compile. The kernels
live in liblokinfer_hip.so (lokinfer_amd/csrc, C-ABI in include/lokinfer_hip.h); there is no other compute path.
"""
from .tensor import DType, Tensor, empty, f16, f32, from_numpy, from_torch, i32, i64, randn, tensor, u8, zeros  # noqa: F401
from . import ops  # noqa: F401
from . import f16_gpu as _f16_gpu
from ._lib import LokinferError, registered_kernels  # noqa: F401
from .compiler import CapturedModel, CompiledModel, Pending, capture, compile, compile_ir, load  # noqa: F401
from .graph import BufferType, Dim, ScalarType, Sym, TensorType, ceildiv  # noqa: F401

ops.f16_gpu = _f16_gpu  # lk.ops.f16_gpu.<name>_f16_gpu, as in the reference

__version__ = "0.1.0"

# A mutable input type: the caller's buffer (a KV cache) written in place, never an output, bound without a copy
# (reference python/lokinfer/types.py: MutableType = BufferType).
MutableType = BufferType


def persistent_buffer(dtype, shape, device: str = "gpu"):
    """Inside a traced graph (lk.compile): model-lifetime state whose contents persist across calls, e.g. a KV
    cache, written in place by kernels declared with `inout` and read like any tensor (reference
    python/lokinfer/__init__.py:26-36). This backend's state starts zeroed; the reference leaves it uninitialized.
    Device "gpu" only: every kernel here runs on the GPU."""
    from .graph import current_graph

    g = current_graph()
    if g is None:
        raise RuntimeError("persistent_buffer() is only valid while tracing a graph (inside lk.compile)")
    if device not in ("cpu", "gpu"):
        raise ValueError("device must be 'cpu' or 'gpu'")
    if device != "gpu":
        raise ValueError("this backend keeps model state on the GPU (device='gpu')")
    return g.persistent(TensorType(dtype, shape), device)


def dim_read(value, index: int = 0, name: str | None = None) -> Dim:
    """Inside a traced graph: reads element `index` of an i32 / i64 tensor at run time into a new symbolic Dim (IR
    dim.read), e.g. a frame count a kernel produced; later ops use it in shapes (reference
    python/lokinfer/ops/view.py:42-58)."""
    from .graph import current_graph

    g = current_graph()
    if g is None:
        raise LokinferError("dim_read is only available while tracing")
    v = g.value_of(value)
    if not isinstance(v.type, TensorType) or v.type.dtype.name not in ("i32", "i64"):
        raise LokinferError("dim_read needs an i32/i64 tensor")
    if not isinstance(index, int) or index < 0:
        raise LokinferError("index must be a non-negative int")
    if name is None:
        name = g.fresh_symbol("R")
    return g.dim_read(v, index, name)
