"""lokinfer_amd: an MI355X-native (CDNA4, gfx950) GPU backend with the lokinfer operator API.

`import lokinfer_amd as lk` gives the reference's front-end names (python/lokinfer/__init__.py in
lariaus/lokinfer): lk.Tensor, lk.from_numpy, lk.randn, lk.f32 / lk.i64, lk.ops.*_gpu, lk.compile. The kernels
live in liblokinfer_hip.so (lokinfer_amd/csrc, C-ABI in include/lokinfer_hip.h); there is no other compute path.
"""
from .tensor import DType, Tensor, empty, f16, f32, from_numpy, from_torch, i32, i64, randn, tensor, u8, zeros  # noqa: F401
from . import ops  # noqa: F401
from . import f16_gpu as _f16_gpu
from ._lib import LokinferError, registered_kernels  # noqa: F401
from .compiler import CapturedModel, CompiledModel, capture, compile, compile_ir, load  # noqa: F401
from .graph import BufferType, Dim, ScalarType, Sym, TensorType  # noqa: F401

ops.f16_gpu = _f16_gpu  # lk.ops.f16_gpu.<name>_f16_gpu, as in the reference

__version__ = "0.1.0"
