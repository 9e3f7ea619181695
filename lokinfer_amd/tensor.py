"""Tensors, dtypes and symbolic types: the reference's `lk.Tensor` / `lk.randn` / `lk.TensorType` surface
(python/lokinfer/tensor.py:11-144, types.py, dims.py in lariaus/lokinfer).

A Tensor wraps a torch tensor that owns the memory: device "gpu" is HIP device memory (cuda:0 in torch-ROCm),
"cpu" is host memory. Unlike the reference's Apple unified memory, the two are distinct and `.to(...)` copies.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass(frozen=True)
class DType:
    name: str
    np: type
    torch: torch.dtype
    size: int


f32 = DType("f32", np.float32, torch.float32, 4)
f16 = DType("f16", np.float16, torch.float16, 2)
i64 = DType("i64", np.int64, torch.int64, 8)
i32 = DType("i32", np.int32, torch.int32, 4)
u8 = DType("u8", np.uint8, torch.uint8, 1)
_BY_TORCH = {d.torch: d for d in (f32, f16, i64, i32, u8)}
_BY_NP = {np.dtype(d.np): d for d in (f32, f16, i64, i32, u8)}


def _torch_device(device: str):
    if device == "gpu":
        return torch.device("cuda", torch.cuda.current_device() if torch.cuda.is_available() else 0)
    if device == "cpu":
        return torch.device("cpu")
    raise ValueError(f"device must be 'cpu' or 'gpu', got {device!r}")


class Tensor:
    """A dense row-major tensor on "cpu" or "gpu"."""

    __slots__ = ("t",)

    def __init__(self, t: torch.Tensor):
        if not t.is_contiguous():
            t = t.contiguous()
        self.t = t

    @property
    def shape(self) -> tuple:
        return tuple(self.t.shape)

    @property
    def dtype(self) -> DType:
        return _BY_TORCH[self.t.dtype]

    @property
    def device(self) -> str:
        return "gpu" if self.t.is_cuda else "cpu"

    @property
    def ndim(self) -> int:
        return self.t.dim()

    @property
    def nbytes(self) -> int:
        return self.t.numel() * self.t.element_size()

    def numel(self) -> int:
        return self.t.numel()

    def data_ptr(self) -> int:
        return self.t.data_ptr()

    def numpy(self) -> np.ndarray:
        """Host copy. For a GPU tensor this is a synchronisation point: a data error a kernel recorded on the
        device (lokinfer_amd._lib.check_device_errors) is raised here as LokinferError."""
        if self.t.is_cuda:
            from ._lib import check_device_errors

            check_device_errors()
        return self.t.detach().cpu().numpy()

    def torch(self, device: str = "cpu") -> torch.Tensor:
        return self.t.to(_torch_device(device))

    def to(self, device: str) -> "Tensor":
        return Tensor(self.t.to(_torch_device(device)))

    def cpu(self) -> "Tensor":
        return self.to("cpu")

    def gpu(self) -> "Tensor":
        return self.to("gpu")

    def tolist(self):
        return self.numpy().tolist()

    def __array__(self, dtype=None, copy=None):
        a = self.numpy()
        return a if dtype is None else a.astype(dtype)

    def __len__(self) -> int:
        return self.shape[0]

    def __repr__(self) -> str:
        return f"lk.Tensor(shape={list(self.shape)}, dtype={self.dtype.name}, device={self.device})"


def from_numpy(a: np.ndarray, device: str = "cpu", copy: bool = False) -> Tensor:
    a = np.ascontiguousarray(a)
    if np.dtype(a.dtype) not in _BY_NP:
        raise TypeError(f"unsupported dtype {a.dtype}")
    t = torch.from_numpy(a.copy() if copy else a)
    return Tensor(t.to(_torch_device(device)) if device != "cpu" else t)


def from_torch(t: torch.Tensor, device: str | None = None, copy: bool = False) -> Tensor:
    if device is not None:
        t = t.to(_torch_device(device))
    return Tensor(t.clone() if copy else t)


def tensor(data, dtype: DType | None = None, device: str = "cpu") -> Tensor:
    a = np.asarray(data, dtype=None if dtype is None else dtype.np)
    return from_numpy(a, device=device, copy=True)


def empty(*shape, dtype: DType = f32, device: str = "cpu") -> Tensor:
    return Tensor(torch.empty(shape, dtype=dtype.torch, device=_torch_device(device)))


def zeros(*shape, dtype: DType = f32, device: str = "cpu") -> Tensor:
    return Tensor(torch.zeros(shape, dtype=dtype.torch, device=_torch_device(device)))


def randn(*shape, dtype: DType = f32, device: str = "cpu", seed: int | None = None) -> Tensor:
    """numpy.random.default_rng(seed).standard_normal(shape) cast to dtype (reference tensor.py:139-144)."""
    rng = np.random.default_rng(seed)
    return from_numpy(rng.standard_normal(shape).astype(dtype.np), device=device, copy=True)
