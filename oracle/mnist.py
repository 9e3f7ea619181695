"""TEST INFRASTRUCTURE ONLY. ctypes binding of oracle/mnist_ref.c (built by oracle/Makefile into
oracle/_build/liblkoracle.so) and the seeded MNIST-MLP inputs of the plumbing config."""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "_build" / "liblkoracle.so"
_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        fp = C.POINTER(C.c_float)
        L.lk_ref_gemm_bias_act_f32.argtypes = [fp, fp, fp, fp, C.c_int64, C.c_int64, C.c_int64, C.c_int]
        L.lk_ref_gemm_bias_act_f32.restype = None
        _lib = L
    return _lib


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def gemm_bias_act(a, b, bias, relu: bool) -> np.ndarray:
    """Bit-exact restatement of gemm_bias[_relu]_f32_cpu (kernels/cpu/gemm.cpp:44-113): per output the k-order
    fma chain, then + bias, then ReLU."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    m, k = a.shape
    n = b.shape[1]
    out = np.empty((m, n), np.float32)
    bp = _fp(np.ascontiguousarray(bias, np.float32)) if bias is not None else None
    lib().lk_ref_gemm_bias_act_f32(_fp(a), _fp(b), bp, _fp(out), m, n, k, 1 if relu else 0)
    return out


# Plumbing config: x[1, 784] ~ N(0, 1); Linear 784->128 + ReLU; Linear 128->10.
# Weights / biases lk.randn(seed) / sqrt(fan_in), i.e. numpy default_rng(seed).standard_normal.
SEEDS = dict(x=1000, w1=1001, b1=1002, w2=1003, b2=1004)


def mlp_inputs(batch: int = 1):
    r = lambda seed, *s: np.random.default_rng(seed).standard_normal(s).astype(np.float32)  # noqa: E731
    x = r(SEEDS["x"], batch, 784)
    w1 = (r(SEEDS["w1"], 784, 128) / np.float32(np.sqrt(784))).astype(np.float32)
    b1 = (r(SEEDS["b1"], 128) / np.float32(np.sqrt(784))).astype(np.float32)
    w2 = (r(SEEDS["w2"], 128, 10) / np.float32(np.sqrt(128))).astype(np.float32)
    b2 = (r(SEEDS["b2"], 10) / np.float32(np.sqrt(128))).astype(np.float32)
    return x, (w1, b1, w2, b2)


def mlp_forward(x, params) -> np.ndarray:
    w1, b1, w2, b2 = params
    return gemm_bias_act(gemm_bias_act(x, w1, b1, True), w2, b2, False)
