"""`lk.ops.f16_gpu`: the reference's f16 GPU op family (python/lokinfer/ops/f16_gpu.py, contracts in
python/lokinfer/ops/f16.py and kernels/gpu/f16_gpu.cpp:1011-1050 in lariaus/lokinfer) on the MI355X kernels of
csrc/f16.hip: the Qwen3-ASR language model's ops. f16 storage, f32 math and accumulation, one rounding to f16 at
each output.

Weights of the GEMM-like ops: the contract fixes the math and leaves the layout to the kernel ("weights may be
pre-packed at build time"). Here a weight w f16[K, N] is packed once into W^T f16[N, K] on the device
(`pack`, a `PackedWeight`); the ops also take a plain f16[K, N] tensor and pack it on the fly (one transpose per
call). The fused SwiGLU ops take [gate | up] concatenated along N, as the reference's `fold_opt` builds it.

Data-dependent errors that the reference's host side reports (an id out of range, more pad ids than audio rows, a
cache write past its end) cannot be raised from a device kernel: rows past the cache are dropped and the other two
give NaN rows (docstrings say which).
"""
from __future__ import annotations

import numpy as np
import torch

from .ops import _launch, check
from .runtime import GpuContext
from .tensor import Tensor, f16, f32, i32, i64

PAD_ID = 151676  # <|audio_pad|> (reference models/qwen3_asr/reference.py)


class PackedWeight:
    """A weight w f16[K, N] packed as W^T f16[N, K] on the device; `shape` is the logical (K, N)."""

    def __init__(self, wt: Tensor):
        check(wt.dtype == f16 and wt.ndim == 2, "packed weight must be f16[N, K]")
        self.wt = wt
        self.shape = (wt.shape[1], wt.shape[0])


def pack(w) -> PackedWeight:
    """w f16[K, N] (numpy array or lk.Tensor) -> PackedWeight (W^T f16[N, K] on the device)."""
    if isinstance(w, PackedWeight):
        return w
    if not isinstance(w, Tensor):
        a = np.ascontiguousarray(w, dtype=np.float16)
        w = Tensor(torch.from_numpy(a).to(GpuContext.shared().device))
    check(w.dtype == f16 and w.ndim == 2, "weight must be f16[K, N]")
    k, n = w.shape
    return PackedWeight(_launch("transpose_f16_gpu", [w], [(n, k)], out_dtypes=[f16]))


def transpose_f16_gpu(w):
    """(MI355X backend) w f16[K, N] -> f16[N, K] (weight packing)."""
    _f16(w, rank=2)
    return _launch("transpose_f16_gpu", [w], [(w.shape[1], w.shape[0])], out_dtypes=[f16])


def _f16(*xs, rank=None):
    for x in xs:
        check(isinstance(x, Tensor) and x.dtype == f16, "expected an f16 tensor")
        if rank is not None:
            check(x.ndim == rank, f"expected rank {rank}, got shape {list(x.shape)}")


def _pos(pos):
    check(isinstance(pos, Tensor) and pos.dtype == i64 and tuple(pos.shape) == (1,), "pos must be i64[1]")


def _w(w) -> PackedWeight:
    return w if isinstance(w, PackedWeight) else pack(w)


def _gemm_rule(x, w):
    _f16(x, rank=2)
    pw = _w(w)
    check(x.shape[1] == pw.shape[0], f"x [M, K] and w [K, N]: inner dims differ: {x.shape}, {pw.shape}")
    check(x.shape[1] % 8 == 0, "K must be a multiple of 8")
    return pw


# ---- GEMM family ------------------------------------------------------------------------------------------

def gemm_f16_gpu(x, w):
    """x f16[M, K] @ w f16[K, N] -> f16[M, N] (f32 accumulation)."""
    pw = _gemm_rule(x, w)
    return _launch("gemm_f16_gpu", [x, pw.wt], [(x.shape[0], pw.shape[1])], out_dtypes=[f16])


def gemm_bias_f16_gpu(x, w, b):
    """x @ w + b (b f16[N])."""
    pw = _gemm_rule(x, w)
    _f16(b, rank=1)
    check(b.shape[0] == pw.shape[1], "b must be f16[N]")
    return _launch("gemm_bias_f16_gpu", [x, pw.wt, b], [(x.shape[0], pw.shape[1])], out_dtypes=[f16])


def gemm_opt_f16_gpu(x, w):
    """x @ w (M = 1: bandwidth-bound GEMV; M > 1: MFMA)."""
    pw = _gemm_rule(x, w)
    return _launch("gemm_opt_f16_gpu", [x, pw.wt], [(x.shape[0], pw.shape[1])], out_dtypes=[f16])


def gemm_bias_opt_f16_gpu(x, w, b):
    """x @ w + b."""
    pw = _gemm_rule(x, w)
    _f16(b, rank=1)
    check(b.shape[0] == pw.shape[1], "b must be f16[N]")
    return _launch("gemm_bias_opt_f16_gpu", [x, pw.wt, b], [(x.shape[0], pw.shape[1])], out_dtypes=[f16])


def gemm_add_opt_f16_gpu(x, w, res):
    """res + x @ w (LM o_proj / down_proj + residual)."""
    pw = _gemm_rule(x, w)
    _f16(res, rank=2)
    check(tuple(res.shape) == (x.shape[0], pw.shape[1]), "res must be f16[M, N]")
    return _launch("gemm_add_opt_f16_gpu", [x, pw.wt, res], [(x.shape[0], pw.shape[1])], out_dtypes=[f16])


def gemm_swiglu_opt_f16_gpu(x, w):
    """y = x f16[M, K] @ w f16[K, 2N] (w = [gate | up]); silu(y[:, :N]) * y[:, N:] -> f16[M, N]."""
    pw = _gemm_rule(x, w)
    check(pw.shape[1] % 2 == 0, "w must be f16[K, 2N] ([gate | up])")
    return _launch("gemm_swiglu_opt_f16_gpu", [x, pw.wt], [(x.shape[0], pw.shape[1] // 2)], out_dtypes=[f16])


def _rms_gemm(name, x, g, w, eps, swiglu):
    pw = _gemm_rule(x, w)
    _f16(g, rank=1)
    check(g.shape[0] == x.shape[1], "g must be f16[K]")
    n = pw.shape[1] // 2 if swiglu else pw.shape[1]
    check(not swiglu or pw.shape[1] % 2 == 0, "w must be f16[K, 2N] ([gate | up])")
    return _launch(name, [x, g, pw.wt], [(x.shape[0], n), tuple(x.shape)], dict(eps=float(eps)),
                   out_dtypes=[f16, f16])


def rmsnorm_gemm_opt_f16_gpu(x, g, w, eps=1e-6):
    """rmsnorm(x, g) @ w -> (y f16[M, N], ws f16[M, K]); ws holds the normalized rows when M > 1 (unspecified at
    M = 1, where one GEMV normalizes the row itself): use y only."""
    return _rms_gemm("rmsnorm_gemm_opt_f16_gpu", x, g, w, eps, False)


def rmsnorm_gemm_swiglu_opt_f16_gpu(x, g, w, eps=1e-6):
    """gemm_swiglu_opt(rmsnorm(x, g), w) -> (y f16[M, N], ws f16[M, K] workspace)."""
    return _rms_gemm("rmsnorm_gemm_swiglu_opt_f16_gpu", x, g, w, eps, True)


def _lm_head(name, x, table):
    _f16(x, table, rank=2)
    check(x.shape[1] == table.shape[1] and x.shape[1] % 8 == 0, "x f16[T, D] and table f16[V, D], D % 8 == 0")
    return _launch(name, [x, table], [(1, table.shape[0])], out_dtypes=[f32])


def lm_head_last_f16_gpu(x, table):
    """Tied LM head on the last row: x[T-1] @ table f16[V, D]^T -> f32[1, V]."""
    return _lm_head("lm_head_last_f16_gpu", x, table)


def lm_head_last_opt_f16_gpu(x, table):
    """lm_head_last (a bandwidth-bound GEMV over the table)."""
    return _lm_head("lm_head_last_opt_f16_gpu", x, table)


# ---- normalization, RoPE, elementwise -----------------------------------------------------------------------

def rmsnorm_f16_gpu(x, g, eps=1e-6):
    """HF Qwen3RMSNorm over the rows of f16[R, C]: h = f16(x rsqrt(mean(x^2) + eps)), y = f16(g h)."""
    _f16(x, rank=2)
    _f16(g, rank=1)
    check(g.shape[0] == x.shape[1] and x.shape[1] % 8 == 0, "g must be f16[C], C % 8 == 0")
    return _launch("rmsnorm_f16_gpu", [x, g], [tuple(x.shape)], dict(eps=float(eps)), out_dtypes=[f16])


def rmsnorm_heads_f16_gpu(x, g, eps=1e-6):
    """rmsnorm over each len(g)-wide head (QK-norm; 128) of f16[R, H hd]."""
    _f16(x, rank=2)
    _f16(g, rank=1)
    check(g.shape[0] % 8 == 0 and x.shape[1] % g.shape[0] == 0, "x must be f16[R, H hd] with g f16[hd], hd % 8 == 0")
    return _launch("rmsnorm_heads_f16_gpu", [x, g], [tuple(x.shape)], dict(eps=float(eps)), out_dtypes=[f16])


def rope_f16_gpu(x, pos, theta=1e6):
    """rotate_half RoPE per 128-wide head of f16[T, H 128] at positions pos + i (pos i64[1] on the device)."""
    _f16(x, rank=2)
    _pos(pos)
    check(x.shape[1] % 128 == 0, "heads must be 128 wide")
    return _launch("rope_f16_gpu", [x, pos], [tuple(x.shape)], dict(theta=float(theta)), out_dtypes=[f16])


def _binary(name, x, y):
    _f16(x, y, rank=2)
    check(tuple(x.shape) == tuple(y.shape), "operands must have the same shape")
    return _launch(name, [x, y], [tuple(x.shape)], out_dtypes=[f16])


def add_f16_gpu(x, y):
    """x + y over f16[R, C]."""
    return _binary("add_f16_gpu", x, y)


def silu_mul_f16_gpu(g, u):
    """g sigmoid(g) u over f16[R, C] (SwiGLU)."""
    return _binary("silu_mul_f16_gpu", g, u)


# ---- embedding, audio scatter, caches, attention ------------------------------------------------------------

def embedding_f16_gpu(ids, table):
    """table[ids]: ids i64[T], table f16[V, D] -> f16[T, D]; an id outside [0, V) gives a NaN row (the reference
    reports a run-time error)."""
    check(isinstance(ids, Tensor) and ids.dtype == i64 and ids.ndim == 1, "ids must be i64[T]")
    _f16(table, rank=2)
    return _launch("embedding_f16_gpu", [ids, table], [(ids.shape[0], table.shape[1])], out_dtypes=[f16])


def scatter_audio_f16_gpu(x, ids, audio, pad_id=PAD_ID):
    """Copy of x f16[T, D] where the j-th row with ids == pad_id becomes audio[j]; a pad row without an audio row
    (more pads than A) is NaN (the reference reports a run-time error)."""
    _f16(x, audio, rank=2)
    check(isinstance(ids, Tensor) and ids.dtype == i64 and tuple(ids.shape) == (x.shape[0],), "ids must be i64[T]")
    check(audio.shape[1] == x.shape[1], "audio must be f16[A, D]")
    return _launch("scatter_audio_f16_gpu", [x, ids, audio], [tuple(x.shape)], dict(pad_id=int(pad_id)),
                   out_dtypes=[f16])


def kv_write_f16_gpu(kc, vc, k, v, pos):
    """kc[pos:pos+T] = k, vc[pos:pos+T] = v (caches f16[cap, D], in place); rows past the cache are dropped."""
    _f16(kc, vc, k, v, rank=2)
    _pos(pos)
    check(tuple(kc.shape) == tuple(vc.shape) and tuple(k.shape) == tuple(v.shape) and k.shape[1] == kc.shape[1],
          "caches f16[cap, D], k / v f16[T, D]")
    check(kc.shape[1] % 8 == 0, "D must be a multiple of 8")
    return _launch("kv_write_f16_gpu", [kc, vc, k, v, pos], [], outs=[], inout=[0, 1])


def _gqa_rule(q, kc, vc, pos, q_heads, kv_heads):
    _f16(q, kc, vc, rank=2)
    _pos(pos)
    check(tuple(kc.shape) == tuple(vc.shape), "caches must both be f16[cap, Dk]")
    check(kv_heads > 0 and q_heads % kv_heads == 0, "q_heads must be a multiple of kv_heads")
    check(q.shape[1] == 128 * q_heads and kc.shape[1] == 128 * kv_heads, "head_dim must be 128")


def attention_gqa_f16_gpu(q, kc, vc, pos, q_heads=16, kv_heads=8):
    """Causal GQA over the cache: query row i of q f16[T, q_heads 128] (position pos + i) attends to cache rows
    0 .. pos + i of its kv head (the caches must already hold them); scale 1/sqrt(128) -> f16[T, q_heads 128]."""
    _gqa_rule(q, kc, vc, pos, q_heads, kv_heads)
    return _launch("attention_gqa_f16_gpu", [q, kc, vc, pos], [tuple(q.shape)],
                   dict(kv_heads=int(kv_heads), q_heads=int(q_heads)), out_dtypes=[f16])


def attention_gqa_opt_f16_gpu(q, kc, vc, pos, q_heads=16, kv_heads=8):
    """attention_gqa (flash tiles on MFMA; key-split chunks for T = 1)."""
    _gqa_rule(q, kc, vc, pos, q_heads, kv_heads)
    return _launch("attention_gqa_opt_f16_gpu", [q, kc, vc, pos], [tuple(q.shape)],
                   dict(kv_heads=int(kv_heads), q_heads=int(q_heads)), out_dtypes=[f16])


def qknorm_rope_kv_opt_f16_gpu(qkv, qg, kg, pos, kc, vc, eps=1e-6, theta=1e6):
    """QK-norm + RoPE + KV write: qkv f16[T, Dq + 2 Dk] (q | k | v). Returns q = rope(rmsnorm_heads(q, qg))
    f16[T, Dq]; writes k = rope(rmsnorm_heads(k, kg)) to kc[pos:pos+T] and v to vc[pos:pos+T] (caches f16[P, Dk], in
    place; the basic composition's roundings kept)."""
    _f16(qkv, kc, vc, rank=2)
    _f16(qg, kg, rank=1)
    _pos(pos)
    check(qg.shape[0] == 128 and kg.shape[0] == 128, "qg / kg must be f16[128]")
    check(tuple(kc.shape) == tuple(vc.shape) and kc.shape[1] % 128 == 0, "caches must both be f16[P, Dk]")
    dq = qkv.shape[1] - 2 * kc.shape[1]
    check(dq > 0 and dq % 128 == 0, "qkv must be f16[T, Dq + 2 Dk] with whole heads")
    return _launch("qknorm_rope_kv_opt_f16_gpu", [qkv, qg, kg, pos, kc, vc], [(qkv.shape[0], dq)],
                   dict(eps=float(eps), theta=float(theta)), out_dtypes=[f16], inout=[4, 5])


# ---- decode-step fusions (MI355X backend) -------------------------------------------------------------------

def attention_decode_qkr_opt_f16_gpu(qkv, qg, kg, pos, kc, vc, counters, eps=1e-6, theta=1e6):
    """(MI355X backend) T = 1: qknorm_rope_kv_opt + attention_gqa_opt in one launch. qkv f16[1, Dq + 2 Dk] ->
    f16[1, Dq]; writes row pos of both caches. counters: i32[Dq / 128] on the device, zero before the first call
    (each call leaves them zero; calls sharing them must be stream-ordered). Bit-identical to the two ops."""
    _f16(qkv, kc, vc, rank=2)
    _f16(qg, kg, rank=1)
    _pos(pos)
    check(qkv.shape[0] == 1, "qkv must be f16[1, W] (one decode row)")
    check(qg.shape[0] == 128 and kg.shape[0] == 128, "qg / kg must be f16[128]")
    check(tuple(kc.shape) == tuple(vc.shape) and kc.shape[1] % 128 == 0, "caches must both be f16[P, Dk]")
    dq = qkv.shape[1] - 2 * kc.shape[1]
    check(dq > 0 and dq % 128 == 0 and (dq // 128) % (kc.shape[1] // 128) == 0, "qkv must be f16[1, Dq + 2 Dk]")
    check(isinstance(counters, Tensor) and counters.dtype == i32 and tuple(counters.shape) == (dq // 128,),
          "counters must be i32[q heads]")
    return _launch("attention_decode_qkr_opt_f16_gpu", [qkv, qg, kg, pos, kc, vc, counters], [(1, dq)],
                   dict(eps=float(eps), theta=float(theta)), out_dtypes=[f16], inout=[4, 5, 6])


def rmsnorm_lm_head_last_opt_f16_gpu(x, g, table, eps=1e-6):
    """(MI355X backend) lm_head_last_opt(rmsnorm(x, g), table): only the last row is normalized, inside the GEMV."""
    _f16(x, table, rank=2)
    _f16(g, rank=1)
    check(x.shape[1] == table.shape[1] == g.shape[0] and x.shape[1] % 8 == 0, "x f16[T, D], g f16[D], table f16[V, D]")
    return _launch("rmsnorm_lm_head_last_opt_f16_gpu", [x, g, table], [(1, table.shape[0])], dict(eps=float(eps)),
                   out_dtypes=[f32])


__all__ = [n for n in dir() if n.endswith("_f16_gpu")] + ["pack", "PackedWeight", "PAD_ID"]
