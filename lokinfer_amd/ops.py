"""`ops.*_gpu`: the reference's GPU kernel ops (python/lokinfer/ops/{gemm,transformer,kokoro_gpu,elementwise,
device}.py in lariaus/lokinfer) with the same names, operand order, attribute names and shape rules, executed
on the MI355X kernels through the C-ABI registry.

Each op checks its operands (OpError, like the reference's `check`), allocates its outputs on the device and
launches the kernel on the current stream. Attributes are passed in attribute-name order: ints/bools as ints,
Python floats as floats (the reference ABI, include/lokinfer/runtime/kernel.h:3-11).

Ops that are not in the reference are marked "(MI355X backend)" in their docstring.

While `lk.compile` traces a function (lokinfer_amd.graph), the same ops record IR instead of launching: operands
are traced values (or captured lk.Tensors), shapes may hold symbolic dims, and the result is a traced value.
"""
from __future__ import annotations

import torch

from . import winograd as _wino
from .graph import TensorType, Value, current_graph
from .runtime import GpuContext
from .tensor import Tensor, f32, i64

STAT_CHUNK = 128


class OpError(ValueError):
    pass


def check(cond: bool, msg: str = "invalid operands") -> None:
    if not cond:
        raise OpError(msg)


def _gpu(*xs: Tensor) -> None:
    for x in xs:
        if isinstance(x, Value):
            continue
        if not isinstance(x, Tensor):
            raise TypeError(f"expected lk.Tensor, got {type(x).__name__}")
        if x.device != "gpu":
            raise OpError("GPU kernel operands must be on the GPU (use ops.to_gpu)")


def _f32(*xs: Tensor, rank: int | None = None) -> None:
    for x in xs:
        check(x.dtype == f32, f"expected f32, got {x.dtype.name}")
        if rank is not None:
            check(x.ndim == rank, f"expected rank {rank}, got shape {list(x.shape)}")


def _launch(name: str, operands: list[Tensor], out_shapes: list[tuple], attrs: dict | None = None,
           out_dtypes: list | None = None, outs: list[Tensor] | None = None, inout: list[int] | None = None):
    """Allocates outputs (unless given) and runs registry kernel `name` with the reference argument layout.
    `inout`: operand indices the kernel writes in place (a KV cache), recorded as the kernel's `inout` attr when
    tracing. While tracing, records the kernel and returns its traced results instead."""
    _gpu(*operands)
    g = current_graph()
    if g is not None:
        if outs:
            raise OpError(f"{name}: writing into a given output cannot be traced; use the op's result")
        kattrs = dict(attrs or {})
        if inout:
            kattrs["inout"] = list(inout)
        out_dtypes = out_dtypes or [f32] * len(out_shapes)
        res = g.kernel(name, list(operands), kattrs, [TensorType(d, s) for s, d in zip(out_shapes, out_dtypes)])
        if not res:
            return None
        return res[0] if len(res) == 1 else tuple(res)
    ctx = GpuContext.shared()
    if outs is None:
        out_dtypes = out_dtypes or [f32] * len(out_shapes)
        outs = [Tensor(torch.empty(s, dtype=d.torch, device=ctx.device)) for s, d in zip(out_shapes, out_dtypes)]
    ints: list[int] = []
    for x in list(operands) + list(outs):
        ints.extend(int(d) for d in x.shape)
    floats: list[float] = []
    for k in sorted(attrs or {}):
        v = attrs[k]
        if isinstance(v, bool) or isinstance(v, int):
            ints.append(int(v))
        elif isinstance(v, float):
            floats.append(v)
        elif isinstance(v, (list, tuple)):
            ints.extend(int(e) for e in v)
        else:
            raise OpError(f"attribute {k}: unsupported type {type(v).__name__}")
    ptrs = [x.data_ptr() for x in list(operands) + list(outs)]
    ctx.run(name, ptrs, ints, floats)
    if not outs:
        return None
    return outs[0] if len(outs) == 1 else tuple(outs)


# ---- device sync (reference ops/device.py:13-25; on discrete HBM these are real copies) ----------------------

def to_gpu(x: Tensor) -> Tensor:
    """Device boundary (reference ops/device.py:13-25). Traced: `sync cpu_to_gpu`, an alias on this runtime (all of
    a model's memory is HBM); eager: a host-to-device copy."""
    g = current_graph()
    if g is not None:
        return g.sync(x, "cpu_to_gpu")
    out = Tensor(x.t.to(GpuContext.shared().device, non_blocking=False))
    return out


def to_cpu(x: Tensor) -> Tensor:
    g = current_graph()
    if g is not None:
        return g.sync(x, "gpu_to_cpu")
    return Tensor(x.t.to("cpu"))


def reshape(x: Tensor, shape) -> Tensor:
    """Zero-cost view with a new shape (same element count)."""
    g = current_graph()
    if g is not None:
        return g.view(x, TensorType(x.dtype, shape), 0)
    return Tensor(x.t.view(*[int(s) for s in shape]))


def view(x: Tensor, shape, offset: int = 0) -> Tensor:
    """Zero-cost view of `shape` starting `offset` elements into x (reference models/kokoro/model.py:109-114)."""
    g = current_graph()
    if g is not None:
        return g.view(x, TensorType(x.dtype, shape), offset)
    n = 1
    for s in shape:
        n *= int(s)
    flat = x.t.reshape(-1)
    check(offset + n <= flat.numel(), "view out of range")
    return Tensor(flat[offset:offset + n].view(*[int(s) for s in shape]))


# ---- GEMM / GEMV --------------------------------------------------------------------------------------------

def _gemm_shapes(a, b, nt=False):
    _f32(a, b, rank=2)
    if nt:
        check(a.shape[1] == b.shape[1], f"gemm_nt: a f32[M, K], b f32[N, K]: {a.shape}, {b.shape}")
        return (a.shape[0], b.shape[0])
    check(a.shape[1] == b.shape[0], f"gemm: a f32[M, K], b f32[K, N]: {a.shape}, {b.shape}")
    return (a.shape[0], b.shape[1])


def gemm_f32_gpu_mps(a, b):
    """a f32[M, K] @ b f32[K, N] -> f32[M, N] (reference ops/gemm.py:32-35)."""
    return _launch("gemm_f32_gpu_mps", [a, b], [_gemm_shapes(a, b)])


def gemm_f32_gpu(a, b):
    return _launch("gemm_f32_gpu", [a, b], [_gemm_shapes(a, b)])


def gemm_nt_f32_gpu_mps(a, b):
    """a f32[M, K] @ b^T (b f32[N, K]) -> f32[M, N] (reference ops/transformer.py:45-48)."""
    return _launch("gemm_nt_f32_gpu_mps", [a, b], [_gemm_shapes(a, b, nt=True)])


def _bias_ok(bias, n):
    _f32(bias, rank=1)
    check(bias.shape[0] == n, "bias must be f32[N]")


def gemm_bias_f32_gpu(a, b, bias):
    s = _gemm_shapes(a, b)
    _bias_ok(bias, s[1])
    return _launch("gemm_bias_f32_gpu", [a, b, bias], [s])


def gemm_bias_relu_f32_gpu(a, b, bias):
    s = _gemm_shapes(a, b)
    _bias_ok(bias, s[1])
    return _launch("gemm_bias_relu_f32_gpu", [a, b, bias], [s])


def gemm_steel_f32_gpu(a, b, bias=None, act="none", residual=None):
    """act(a @ b + bias) [+ residual] (reference ops/transformer.py:166-180)."""
    s = _gemm_shapes(a, b)
    if bias is None:
        check(act == "none" and residual is None, "act / residual need a bias")
        return _launch("gemm_steel_f32_gpu", [a, b], [s])
    _bias_ok(bias, s[1])
    if residual is not None:
        check(act == "none" and tuple(residual.shape) == s, "residual must be f32[M, N], act none")
        return _launch("gemm_steel_bias_res_f32_gpu", [a, b, bias, residual], [s])
    name = {"none": "gemm_steel_bias_f32_gpu", "gelu": "gemm_steel_bias_gelu_f32_gpu",
            "relu": "gemm_steel_bias_relu_f32_gpu"}[act]
    return _launch(name, [a, b, bias], [s])


def gemm_nt_steel_f32_gpu(a, b):
    return _launch("gemm_nt_steel_f32_gpu", [a, b], [_gemm_shapes(a, b, nt=True)])


def _gemv_shapes(x, w, bias=None):
    _f32(x, w, rank=2)
    check(x.shape[0] == 1 and x.shape[1] == w.shape[0], f"x must be f32[1, K] and w f32[K, N]: {x.shape}, {w.shape}")
    if bias is not None:
        _bias_ok(bias, w.shape[1])
    return (1, w.shape[1])


def gemv4_f32_gpu(x, w, bias=None, act="none", residual=None, cw=0):
    """x f32[1, K] @ w f32[K, N] (+ bias) (gelu) (+ residual) -> f32[1, N] (reference ops/transformer.py:371-382).
    cw (Metal column width) is accepted and ignored: the CDNA4 kernel picks its own K split."""
    check(cw in (0, 2, 4, 8, 16), "cw must be 0 (auto), 2, 4, 8 or 16")
    s = _gemv_shapes(x, w, bias)
    check(w.shape[1] % 4 == 0, "N must be a multiple of 4")
    if bias is None:
        check(act == "none" and residual is None, "act / residual need a bias")
        return _launch("gemv4_f32_gpu", [x, w], [s], dict(cw=cw))
    if residual is not None:
        check(tuple(residual.shape) == s, "residual must be f32[1, N]")
        return _launch("gemv4_bias_res_f32_gpu", [x, w, bias, residual], [s], dict(cw=cw))
    name = "gemv4_bias_gelu_f32_gpu" if act == "gelu" else "gemv4_bias_f32_gpu"
    return _launch(name, [x, w, bias], [s], dict(cw=cw))


def gemv_f32_gpu(x, w, bias=None, act="none"):
    s = _gemv_shapes(x, w, bias)
    if bias is None:
        check(act == "none", "act needs a bias")
        return _launch("gemv_f32_gpu", [x, w], [s])
    return _launch("gemv_bias_gelu_f32_gpu" if act == "gelu" else "gemv_bias_f32_gpu", [x, w, bias], [s])


def gemv_rows_f32_gpu(x, w):
    """x f32[1, K] . rows of w f32[N, K] -> f32[1, N] (tied LM head; reference ops/transformer.py:209-215)."""
    _f32(x, w, rank=2)
    check(x.shape[0] == 1 and x.shape[1] == w.shape[1], "x must be f32[1, K] and w f32[N, K]")
    return _launch("gemv_rows_f32_gpu", [x, w], [(1, w.shape[0])])


def gemv1_bias_f32_gpu(x, w, b):
    """x f32[R, K] @ w f32[K, 1] + b f32[1] -> f32[R, 1] (reference gemv1_bias, kokoro_lc.cpp:257-267)."""
    _f32(x, w, rank=2)
    check(w.shape == (x.shape[1], 1) and tuple(b.shape) == (1,), "w must be f32[K, 1], b f32[1]")
    return _launch("gemv1_bias_f32_gpu", [x, w, b], [(x.shape[0], 1)])


# ---- conv1d (channel-last) ----------------------------------------------------------------------------------

def _conv_lc_shape(x, w, b, padding, dilation, stride):
    _f32(x, rank=2)
    _f32(w, rank=3)
    _f32(b, rank=1)
    check(w.shape[2] == x.shape[1], f"w must be [Co, K, Ci]: x {x.shape}, w {w.shape}")
    check(b.shape[0] == w.shape[0], "bias must be f32[Co]")
    check(x.shape[1] % 16 == 0, "Ci must be a multiple of 16")
    check(stride >= 1 and dilation >= 1 and padding >= 0, "invalid conv attrs")
    lo = (x.shape[0] + 2 * padding - dilation * (w.shape[1] - 1) - 1) // stride + 1
    check(lo >= 1, "empty conv output")
    return (lo, w.shape[0])


def conv1d_lc_f32_gpu(x, w, b, residual=None, out_scale=1.0, padding=0, dilation=1, stride=1):
    """(conv1d(x, w) + b [+ residual]) * out_scale, channel-last: x f32[L, Ci], w f32[Co, K, Ci] -> f32[Lo, Co]
    (reference ops/kokoro_gpu.py:20-54). stride > 1 is an MI355X-backend extension (the reference keeps strided
    convs on the CPU)."""
    s = _conv_lc_shape(x, w, b, padding, dilation, stride)
    attrs = dict(padding=int(padding), dilation=int(dilation), stride=int(stride))
    if residual is None:
        check(out_scale == 1.0, "out_scale needs a residual")
        return _launch("conv1d_lc_f32_gpu", [x, w, b], [s], attrs)
    check(tuple(residual.shape) == s, "residual shape mismatch")
    return _launch("conv1d_lc_res_f32_gpu", [x, w, b, residual], [s], dict(attrs, oscale=float(out_scale)))


def conv1d_act_lc_f32_gpu(x, w, b, affine, alpha=None, act="snake", slope=0.0, residual=None, out_scale=1.0,
                          padding=0, dilation=1, stride=1, stats=False):
    """(MI355X backend) conv1d_lc over act(affine(x)) with the prologue fused into the implicit-GEMM operand
    staging: v = (x - af[0]) * af[1] + af[2] per channel, then snake(alpha) / leaky(slope) / none; the conv's zero
    padding applies after the activation. Replaces the reference's snake_affine_lc + conv1d_lc pair and its
    Winograd transform prologue (winograd.metal:37-91)."""
    s = _conv_lc_shape(x, w, b, padding, dilation, stride)
    _f32(affine, rank=2)
    check(affine.shape == (3, x.shape[1]), "affine must be f32[3, Ci]")
    code = {"none": 0, "snake": 1, "leaky": 2}[act]
    if alpha is None:
        check(code != 1, "snake needs alpha")
        alpha = b  # unused operand slot
    check(alpha.shape[0] == x.shape[1] or code != 1, "alpha must be f32[Ci]")
    attrs = dict(act=code, dilation=int(dilation), oscale=float(out_scale), padding=int(padding), slope=float(slope),
                 stride=int(stride))
    # stats=True also returns the output's per-(128-row chunk, channel) (mean, M2), the channel_stats_lc layout,
    # computed in the conv's epilogue
    shapes = [s, (-(-s[0] // STAT_CHUNK), s[1], 2)] if stats else [s]
    sfx = "_stats" if stats else ""
    if residual is None:
        check(out_scale == 1.0, "out_scale needs a residual")
        return _launch(f"conv1d_act_lc{sfx}_f32_gpu", [x, w, b, affine, alpha], shapes, attrs)
    check(tuple(residual.shape) == s, "residual shape mismatch")
    return _launch(f"conv1d_act_lc_res{sfx}_f32_gpu", [x, w, b, affine, alpha, residual], shapes, attrs)


# ---- Winograd / Toom-Cook conv1d (reference ops/winograd.py:98-247) ------------------------------------------
# x [L, Ci] -> V [d * A * rmax, Ci] (input transform, activation fused) -> per point a GEMM V_xi . U_xi over
# (group, ci) with the AT output transform, bias, [residual * scale] and [128-row channel statistics] in the
# epilogue. U and tr come from winograd.wino_weights(w) on the host, once per weight.

def _wino_lo(x, kernel, dilation, padding):
    lo = x.shape[0] + 2 * padding - dilation * (kernel - 1)
    check(lo >= 1, "empty conv output")
    return lo


def _wino_attrs_ok(x, dilation, groups, kernel, padding, tile):
    _f32(x, rank=2)
    check(x.shape[1] % 16 == 0, "Ci must be a multiple of 16")
    check((tile == _wino.TILE or (tile == 2 and kernel == 3)) and _wino.variant(kernel)[1] == groups,
          "groups / tile don't match the kernel size")
    check(dilation >= 1 and padding >= 0 and padding % dilation == 0, "padding must be a multiple of dilation")


def _wino_v_shape(x, dilation, groups, kernel, padding, tile):
    _wino_attrs_ok(x, dilation, groups, kernel, padding, tile)
    lo = _wino_lo(x, kernel, dilation, padding)
    return (_wino.tiles_rows(lo, dilation, groups, tile, kernel), x.shape[1])


def wino_tf_lc_f32_gpu(x, tr, dilation, groups, kernel, padding, tile, affine=None, alpha=None, slope=None):
    """Input transform V[rho, xi, r, c] = sum_j BT[xi, j] h[rho + d (r M + j) - pad] of h = x, or of snake(affine(x))
    (affine and alpha) / leaky(affine(x), slope) (affine and slope). Reference winograd.py:128-154."""
    s = _wino_v_shape(x, dilation, groups, kernel, padding, tile)
    a = _wino.alpha_of(kernel, tile)
    _f32(tr, rank=1)
    check(tr.shape[0] == a * (a + tile), "bad transform table")
    attrs = dict(dilation=int(dilation), groups=int(groups), kernel=int(kernel), padding=int(padding), tile=int(tile))
    if affine is None:
        return _launch("wino_tf_lc_f32_gpu", [x, tr], [s], attrs)
    _f32(affine, rank=2)
    check(affine.shape == (3, x.shape[1]), "affine must be f32[3, C]")
    if slope is not None:
        check(alpha is None, "give either alpha (snake) or slope (leaky)")
        return _launch("wino_tf_leaky_lc_f32_gpu", [x, tr, affine], [s], dict(attrs, slope=float(slope)))
    check(alpha is not None and alpha.shape == (x.shape[1],), "alpha must be f32[C]")
    return _launch("wino_tf_snake_lc_f32_gpu", [x, tr, affine, alpha], [s], attrs)


def wino_mm_lc_f32_gpu(v, u, b, tr, x, dilation, groups, kernel, padding, tile, residual=None, out_scale=1.0,
                       stats=False, u_layout=0):
    """Per-point GEMM + AT output transform + bias [+ residual * out_scale] [+ per-128-row channel (mean, M2)],
    out [Lo, Co], stats [d * chunks, Co, 2]. Reference winograd.py:157-202. u_layout = 1 (MI355X backend): u is
    U tiled, f32[A, Co / 64, groups * Ci * 64] (winograd.wino_weights_t), the same result."""
    _wino_attrs_ok(x, dilation, groups, kernel, padding, tile)
    _f32(v, rank=2)
    _f32(u, rank=3)
    _f32(b, tr, rank=1)
    check(u_layout in (0, 1), "u_layout must be 0 or 1")
    a, nci, co = (u.shape[0], u.shape[2] // 64, u.shape[1] * 64) if u_layout else u.shape
    check(a == _wino.alpha_of(kernel, tile), "u must come from wino_weights for this kernel size")
    check(nci == groups * x.shape[1] and (not u_layout or u.shape[2] % 64 == 0),
          "u must be f32[A, groups * Ci, Co] (u_layout 1: [A, Co / 64, groups * Ci * 64])")
    check(co % 64 == 0, "Co must be a multiple of 64")
    check(b.shape[0] == co, "bias must be f32[Co]")
    check(tr.shape[0] == a * (a + tile), "bad transform table")
    check(tuple(v.shape) == _wino_v_shape(x, dilation, groups, kernel, padding, tile), "v must be wino_tf of x")
    lo = _wino_lo(x, kernel, dilation, padding)
    shapes = [(lo, co)]
    if stats:
        shapes.append((_wino.stats_chunks(lo, dilation) * dilation, co, 2))
    attrs = dict(dilation=int(dilation), groups=int(groups), kernel=int(kernel), padding=int(padding), tile=int(tile))
    if u_layout:
        attrs["u_layout"] = 1
    sfx = "_stats" if stats else ""
    if residual is None:
        check(out_scale == 1.0, "out_scale needs a residual")
        return _launch(f"wino_mm{sfx}_lc_f32_gpu", [v, u, b, tr, x], shapes, attrs)
    _f32(residual, rank=2)
    check(tuple(residual.shape) == (lo, co), "residual shape mismatch")
    return _launch(f"wino_mm_res{sfx}_lc_f32_gpu", [v, u, b, tr, x, residual], shapes,
                   dict(attrs, oscale=float(out_scale)))


def wino_adain_affine_lc_f32_gpu(stats, gb, length, dilation=1, eps=1e-5):
    """AdaIN affine f32[3, C] = (mean, (1 + g) / std, b) from the Winograd epilogue statistics over `length` output
    rows (chunk i = (rho, y), rows clamp(ceil((length - rho) / d) - 128 y, 0, 128)); channels >= Creal get 0.
    Reference winograd.py:204-218."""
    _f32(stats, rank=3)
    _f32(gb, rank=1)
    check(stats.shape[2] == 2, "stats must be f32[S, C, 2]")
    check(gb.shape[0] % 2 == 0 and gb.shape[0] // 2 <= stats.shape[1], "gb must be f32[2 Creal] with Creal <= C")
    check(stats.shape[0] == _wino.stats_chunks(int(length), dilation) * dilation, "stats chunks don't match length")
    return _launch("wino_adain_affine_lc_f32_gpu", [stats, gb], [(3, stats.shape[1])],
                   dict(dilation=int(dilation), eps=float(eps), length=int(length)))


def conv1d_wino_lc_f32_gpu(x, u, b, tr, kernel, residual=None, out_scale=1.0, padding=0, dilation=1, affine=None,
                           alpha=None, slope=None, stats=False, u_layout=0):
    """(conv1d(h, w) + b [+ residual]) * out_scale with (u, tr) = winograd.wino_weights(w), h = x, or
    snake(affine(x), alpha), or leaky(affine(x), slope); stats=True also returns the output's channel statistics
    for wino_adain_affine_lc_f32_gpu. Two launches: transform, GEMM. Reference winograd.py:221-247."""
    kernel = int(kernel)
    _, n = _wino.variant(kernel)
    tile = 2 if u.shape[0] == 4 else _wino.TILE
    attrs = dict(dilation=int(dilation), groups=n, kernel=kernel, padding=int(padding), tile=tile)
    if affine is None:
        check(alpha is None and slope is None, "alpha / slope need an affine")
    v = wino_tf_lc_f32_gpu(x, tr, affine=affine, alpha=alpha, slope=slope, **attrs)
    return wino_mm_lc_f32_gpu(v, u, b, tr, x, residual=residual, out_scale=out_scale, stats=stats, u_layout=u_layout,
                              **attrs)


# ---- transformer --------------------------------------------------------------------------------------------

def layernorm_f32_gpu(x, gamma, beta, eps=1e-5):
    _f32(x, rank=2)
    check(x.shape[1] <= 2048 and gamma.shape == (x.shape[1],) and beta.shape == (x.shape[1],), "layernorm: bad shapes")
    return _launch("layernorm_f32_gpu", [x, gamma, beta], [x.shape], dict(eps=float(eps)))


def _abln_check(a, bias, r, gamma, beta):
    _f32(a, r, rank=2)
    check(tuple(a.shape) == tuple(r.shape), "residual shape mismatch")
    check(a.shape[1] <= 2048, "C must be <= 2048")
    check(all(tuple(v.shape) == (a.shape[1],) for v in (bias, gamma, beta)), "bias/gamma/beta must be f32[C]")


def add_bias_layernorm_f32_gpu(a, bias, r, gamma, beta, eps=1e-12):
    """LayerNorm(a + bias + r) * gamma + beta (reference ops/kokoro_gpu.py:273-295)."""
    _abln_check(a, bias, r, gamma, beta)
    return _launch("add_bias_layernorm_f32_gpu", [a, bias, r, gamma, beta], [a.shape], dict(eps=float(eps)))


def add_bias_layernorm2_f32_gpu(a, bias, r, gamma, beta, eps=1e-5):
    """(s, LN(s)) with s = a + bias + r (reference ops/transformer.py:51-64)."""
    _abln_check(a, bias, r, gamma, beta)
    return _launch("add_bias_layernorm2_f32_gpu", [a, bias, r, gamma, beta], [a.shape, a.shape], dict(eps=float(eps)))


def bias_gelu_f32_gpu(x, bias):
    _f32(x, rank=2)
    _bias_ok(bias, x.shape[1])
    return _launch("bias_gelu_f32_gpu", [x, bias], [x.shape])


def _attn_shape(qkv, bias, heads):
    _f32(qkv, rank=2)
    check(qkv.shape[1] == 3 * 64 * heads, "qkv must be f32[T, 3D] with head_dim = 64")
    check(tuple(bias.shape) == (qkv.shape[1],), "bias must be f32[3D]")
    return (qkv.shape[0], qkv.shape[1] // 3)


def attention_qkv_f32_gpu(qkv, bias, heads, causal=False):
    s = _attn_shape(qkv, bias, heads)
    return _launch("attention_qkv_causal_f32_gpu" if causal else "attention_qkv_f32_gpu", [qkv, bias], [s],
                  dict(heads=int(heads)))


def attention_qkv_sg_f32_gpu(qkv, bias, heads, causal=False, nsg=4):
    """Flash SDPA over fused QKV + bias (reference ops/transformer.py:297-307); nsg is a Metal launch shape and is
    accepted for ABI compatibility."""
    s = _attn_shape(qkv, bias, heads)
    return _launch("attention_qkv_sg_causal_f32_gpu" if causal else "attention_qkv_sg_f32_gpu", [qkv, bias], [s],
                  dict(heads=int(heads), nsg=int(nsg)))


def _decode_check(qkv, kc, vc, pos, bias, heads):
    _f32(qkv, kc, vc, rank=2)
    d = kc.shape[1]
    check(qkv.shape == (1, 3 * d) and vc.shape == kc.shape and d == 64 * heads, "decode attention: bad shapes")
    check(pos.dtype == i64 and tuple(pos.shape) == (1,), "pos must be i64[1]")
    check(tuple(bias.shape) == (3 * d,), "bias must be f32[3D]")
    _gpu(pos)
    return (1, d)


def attention_decode_split_f32_gpu(qkv, kcache, vcache, pos, bias, heads, splits=0, nsg=0, single=1):
    """Writes k, v (+ bias) at row pos of the caches (in place) and attends one query over rows 0..pos
    (reference ops/transformer.py:323-337). pos is a device i64[1]; the caller guarantees pos < cache rows."""
    s = _decode_check(qkv, kcache, vcache, pos, bias, heads)
    return _launch("attention_decode_split_f32_gpu", [qkv, kcache, vcache, pos, bias], [s],
                  dict(heads=int(heads), nsg=int(nsg), single=int(single), splits=int(splits)), inout=[1, 2])


# ---- fused decode step (backend ops; they replace one layer's gemv4 / attention_decode_split /
# add_bias_layernorm2 sequence, reference ops/transformer.py:51-64, 323-382) ------------------------------------

def gemv_partial_slices(k: int) -> int:
    """Row slices of a partial GEMV over K (16 rows per wave up to K = 1024, else 64)."""
    rpw = 16 if k <= 1024 else 64
    return -(-int(k) // (4 * rpw))


def gemv_partial_f32_gpu(x, w):
    """Row-slice partial sums of x f32[1, K] @ w f32[K, N] -> f32[S, N], S = gemv_partial_slices(K); the slices
    are summed (in order) by the consuming op."""
    _f32(x, w, rank=2)
    check(x.shape[0] == 1 and x.shape[1] == w.shape[0], "x must be f32[1, K] and w f32[K, N]")
    check(w.shape[1] % 4 == 0, "N must be a multiple of 4")
    return _launch("gemv_partial_f32_gpu", [x, w], [(gemv_partial_slices(w.shape[0]), w.shape[1])])


def gemv_partial_gelu_f32_gpu(xpart, xbias, w):
    """Partial GEMV whose input is gelu_tanh(sum of the slices of xpart f32[Sx, K] + xbias f32[K])."""
    _f32(xpart, w, rank=2)
    k = xpart.shape[1]
    check(w.shape[0] == k and w.shape[1] % 4 == 0, "w must be f32[K, N] with N % 4 == 0")
    _bias_ok(xbias, k)
    return _launch("gemv_partial_gelu_f32_gpu", [xpart, xbias, w], [(gemv_partial_slices(k), w.shape[1])])


def gemv_partial_attn_f32_gpu(chunks, w):
    """Partial GEMV whose input is the merged decode attention of chunks f32[H, C, 66] (64 dims per head)."""
    _f32(chunks, rank=3)
    _f32(w, rank=2)
    check(chunks.shape[2] == 66 and w.shape[0] == 64 * chunks.shape[0] and w.shape[1] % 4 == 0,
          "expected chunks [H, C, 66] and w [64 H, N], N % 4 == 0")
    return _launch("gemv_partial_attn_f32_gpu", [chunks, w], [(gemv_partial_slices(w.shape[0]), w.shape[1])])


def gemv_partial_res_ln_f32_gpu(xpart, xbias, res, gamma, beta, w, eps=1e-5):
    """(part, s): partial GEMV of LN(s) with s = (slices of xpart f32[Sx, K]) + xbias + res f32[1, K], K <= 1024;
    s is returned as the new residual stream."""
    _f32(xpart, res, w, rank=2)
    k = xpart.shape[1]
    check(tuple(res.shape) == (1, k) and w.shape[0] == k and w.shape[1] % 4 == 0 and k <= 1024 and k % 4 == 0,
          "expected res [1, K], w [K, N] with N % 4 == 0, K % 4 == 0, K <= 1024")
    for v in (xbias, gamma, beta):
        _bias_ok(v, k)
    return _launch("gemv_partial_res_ln_f32_gpu", [xpart, xbias, res, gamma, beta, w],
                   [(gemv_partial_slices(k), w.shape[1]), (1, k)], dict(eps=float(eps)))


def gemv_partial_ln_f32_gpu(x, gamma, beta, w, eps=1e-5):
    """(part, x'): partial GEMV of LN(x) for x f32[1, K], K <= 1024 (x' is a copy of x)."""
    _f32(x, w, rank=2)
    k = x.shape[1]
    check(x.shape[0] == 1 and w.shape[0] == k and w.shape[1] % 4 == 0 and k <= 1024 and k % 4 == 0,
          "expected x [1, K], w [K, N] with N % 4 == 0, K % 4 == 0, K <= 1024")
    for v in (gamma, beta):
        _bias_ok(v, k)
    return _launch("gemv_partial_ln_f32_gpu", [x, gamma, beta, w], [(gemv_partial_slices(k), w.shape[1]), (1, k)],
                   dict(eps=float(eps)))


def gemv_partial_embed_ln_f32_gpu(table, ids, table2, ids2, gamma, beta, w, eps=1e-5):
    """(part, s): partial GEMV of LN(s) with s = table[ids] + table2[ids2] f32[1, K] (the layer-0 prologue of a
    decode step: token + position embedding, LayerNorm, first GEMV); s is returned as the residual stream."""
    _f32(table, table2, w, rank=2)
    k = table.shape[1]
    check(table2.shape[1] == k and w.shape[0] == k and w.shape[1] % 4 == 0 and k <= 1024 and k % 4 == 0,
          "expected table [V, K], table2 [P, K], w [K, N] with N % 4 == 0, K % 4 == 0, K <= 1024")
    for ix in (ids, ids2):
        check(ix.dtype == i64 and tuple(ix.shape) == (1,), "ids must be i64[1]")
    for v in (gamma, beta):
        _bias_ok(v, k)
    return _launch("gemv_partial_embed_ln_f32_gpu", [table, ids, table2, ids2, gamma, beta, w],
                   [(gemv_partial_slices(k), w.shape[1]), (1, k)], dict(eps=float(eps)))


def lm_head_ln_argmax_f32_gpu(part, bias, res, gamma, beta, table, eps=1e-5):
    """(logits f32[1, V], argmax i64[1]): logits = LN(s) @ table^T with s = (slices of part f32[S, K]) + bias + res
    (final LayerNorm + tied LM head + greedy argmax of a decode step); argmax is the first index of the maximum."""
    _f32(part, res, table, rank=2)
    k = part.shape[1]
    check(tuple(res.shape) == (1, k) and table.shape[1] == k and k <= 1024 and k % 4 == 0,
          "expected part [S, K], res [1, K], table [V, K], K % 4 == 0, K <= 1024")
    for v in (bias, gamma, beta):
        _bias_ok(v, k)
    return _launch("lm_head_ln_argmax_f32_gpu", [part, bias, res, gamma, beta, table], [(1, table.shape[0]), (1,)],
                   dict(eps=float(eps)), out_dtypes=[f32, i64])


def attention_decode_part_f32_gpu(qkv_part, kcache, vcache, pos, bias, heads):
    """Decode attention over cache rows 0..pos with q, k, v = slice sums of qkv_part f32[S, 3D] + bias; writes
    row pos of both caches (in place) and returns the per-(head, 64-key chunk) partials f32[H, C, 66]."""
    _f32(qkv_part, kcache, vcache, rank=2)
    d = kcache.shape[1]
    check(qkv_part.shape[1] == 3 * d and vcache.shape == kcache.shape and d == 64 * heads, "bad decode shapes")
    check(pos.dtype == i64 and tuple(pos.shape) == (1,), "pos must be i64[1]")
    check(tuple(bias.shape) == (3 * d,), "bias must be f32[3D]")
    chunks = -(-kcache.shape[0] // 64)
    return _launch("attention_decode_part_f32_gpu", [qkv_part, kcache, vcache, pos, bias], [(heads, chunks, 66)],
                   dict(heads=int(heads)), inout=[1, 2])


def reduce_bias_res_ln2_f32_gpu(part, bias, res, gamma, beta, eps=1e-5):
    """(s, LN(s)) with s = (sum of the slices of part f32[S, N]) + bias + res; N <= 1024."""
    _f32(part, res, rank=2)
    n = part.shape[1]
    check(tuple(res.shape) == (1, n), "res must be f32[1, N]")
    for v in (bias, gamma, beta):
        _bias_ok(v, n)
    return _launch("reduce_bias_res_ln2_f32_gpu", [part, bias, res, gamma, beta], [(1, n), (1, n)],
                   dict(eps=float(eps)))


def attention_decode_kvw_f32_gpu(qkv, kcache, vcache, pos, bias, heads):
    s = _decode_check(qkv, kcache, vcache, pos, bias, heads)
    return _launch("attention_decode_kvw_f32_gpu", [qkv, kcache, vcache, pos, bias], [s], dict(heads=int(heads)),
                   inout=[1, 2])


def attention_decode_f32_gpu(qkv, kcache, vcache, pos, bias, heads):
    s = _decode_check(qkv, kcache, vcache, pos, bias, heads)
    return _launch("attention_decode_f32_gpu", [qkv, kcache, vcache, pos, bias], [s], dict(heads=int(heads)))


def kv_write_f32_gpu(kcache, vcache, qkv, pos, bias):
    _decode_check(qkv, kcache, vcache, pos, bias, kcache.shape[1] // 64)
    return _launch("kv_write_f32_gpu", [kcache, vcache, qkv, pos, bias], [], outs=[], inout=[0, 1])


# ---- chunked prefill / generate (reference python/lokinfer/ops/transformer.py:220-282, 348-351, 441-517) ------

def _rows_check(kc, vc, qkv, pos, bias):
    _f32(kc, vc, qkv, rank=2)
    check(kc.shape == vc.shape, "caches must be f32[P, D]")
    check(qkv.shape[1] == 3 * kc.shape[1], "qkv must be f32[T, 3D]")
    check(pos.dtype == i64 and tuple(pos.shape) == (1,), "pos must be i64[1] (start position)")
    _f32(bias, rank=1)
    check(bias.shape[0] == qkv.shape[1], "bias must be f32[3D]")
    _gpu(pos)


def kv_write_rows_f32_gpu(kcache, vcache, qkv, pos, bias):
    """kcache[pos + i] = k_i + bk, vcache[pos + i] = v_i + bv for the T rows of qkv f32[T, 3D]; in place. pos is a
    device i64[1]; rows at or past the cache's end are dropped (the reference reports an error on the host)."""
    _rows_check(kcache, vcache, qkv, pos, bias)
    check(kcache.shape[1] % 4 == 0, "D must be a multiple of 4")
    return _launch("kv_write_rows_f32_gpu", [kcache, vcache, qkv, pos, bias], [], outs=[], inout=[0, 1])


def _cache_attn(name, qkv, kcache, vcache, pos, bias, heads, attrs):
    _rows_check(kcache, vcache, qkv, pos, bias)
    check(kcache.shape[1] == 64 * int(heads), "head_dim must be 64")
    writes = name.startswith("attention_gen")  # the gen ops write the chunk's rows into the caches
    return _launch(name, [qkv, kcache, vcache, pos, bias], [(qkv.shape[0], kcache.shape[1])], attrs,
                   inout=[1, 2] if writes else None)


def attention_cache_f32_gpu(qkv, kcache, vcache, pos, bias, heads):
    """Causal attention of the T queries of qkv f32[T, 3D] (positions pos .. pos+T-1, q bias added) over cache rows
    0 .. pos+i, which must already hold the chunk's k / v (kv_write_rows) -> f32[T, D]; head_dim 64, scale 1/8."""
    return _cache_attn("attention_cache_f32_gpu", qkv, kcache, vcache, pos, bias, heads, dict(heads=int(heads)))


def attention_cache_sg_f32_gpu(qkv, kcache, vcache, pos, bias, heads, nsg=4):
    """attention_cache_f32_gpu; nsg (the reference's simdgroups per threadgroup: 2, 4, 8) is validated and has no
    meaning on CDNA4, where one MFMA kernel serves both."""
    check(int(nsg) in (2, 4, 8), "nsg must be 2, 4 or 8")
    return _cache_attn("attention_cache_sg_f32_gpu", qkv, kcache, vcache, pos, bias, heads,
                       dict(heads=int(heads), nsg=int(nsg)))


def attention_gen_f32_gpu(qkv, kcache, vcache, pos, bias, heads):
    """Writes the T new k / v rows (+ bias) at pos.. (in place) and attends causally over rows 0..pos+i: T = 1 -> the
    split-key decode attention, T > 1 -> kv_write_rows + attention_cache."""
    return _cache_attn("attention_gen_f32_gpu", qkv, kcache, vcache, pos, bias, heads, dict(heads=int(heads)))


def attention_gen2_f32_gpu(qkv, kcache, vcache, pos, bias, heads):
    """attention_gen_f32_gpu (the reference's second kernel set; on CDNA4 both names run the same kernels)."""
    return _cache_attn("attention_gen2_f32_gpu", qkv, kcache, vcache, pos, bias, heads, dict(heads=int(heads)))


def _splitk_check(a, b, splits, tile):
    _f32(a, b, rank=2)
    check(a.shape[1] == b.shape[0], "inner dimensions differ")
    check(int(splits) >= 1 and a.shape[1] % (16 * int(splits)) == 0, "K must be divisible by 16*splits")
    check(int(tile) in (32, 64), "tile must be 32 or 64")
    check(b.shape[1] % 4 == 0, "N must be a multiple of 4")
    return (int(splits), a.shape[0], b.shape[1])


def gemm_splitk_f32_gpu(a, b, splits, tile=64):
    """Split-K partials f32[S, M, N], part s = a[:, sK/S:(s+1)K/S] @ b[sK/S:(s+1)K/S, :], consumed by
    add_bias_layernorm2_sk_f32_gpu. While the output tiles fill the GPU (and for M = 1) only plane 0 is written,
    holding the whole product, and the consumer reads only that plane (rule splitk_planes)."""
    s = _splitk_check(a, b, splits, tile)
    return _launch("gemm_splitk_f32_gpu", [a, b], [s], dict(splits=int(splits), tile=int(tile)))


def gemm_auto_sk_f32_gpu(a, b, splits, tile=32):
    """gemm_splitk_f32_gpu for a graph serving T = 1 and T > 1: M = 1 -> GEMV into plane 0."""
    s = _splitk_check(a, b, splits, tile)
    return _launch("gemm_auto_sk_f32_gpu", [a, b], [s], dict(splits=int(splits), tile=int(tile)))


SPLITK_MAX_TILES = 64


def splitk_planes(m: int, n: int, splits: int) -> int:
    """Planes of a split-K partial tensor that hold data: splits while M > 1 and the 64 x 64 output tiles number
    fewer than SPLITK_MAX_TILES, else 1."""
    return splits if m > 1 and (-(-m // 64)) * (-(-n // 64)) < SPLITK_MAX_TILES else 1


def add_bias_layernorm2_sk_f32_gpu(parts, bias, r, gamma, beta, eps=1e-5):
    """add_bias_layernorm2_f32_gpu with a = the sum of the split-K partials parts f32[S, R, C] -> (sum, LN(sum))."""
    _f32(parts, rank=3)
    _f32(r, rank=2)
    _f32(bias, gamma, beta, rank=1)
    check(tuple(parts.shape[1:]) == tuple(r.shape), "parts must be f32[S, R, C] over r f32[R, C]")
    check(r.shape[1] <= 2048 and bias.shape[0] == gamma.shape[0] == beta.shape[0] == r.shape[1], "C must be <= 2048")
    return _launch("add_bias_layernorm2_sk_f32_gpu", [parts, bias, r, gamma, beta], [tuple(r.shape)] * 2,
                   dict(eps=float(eps)))


def gemm_auto_f32_gpu(x, w):
    """x f32[M, K] @ w f32[K, N]: M = 1 -> GEMV (decode), else the MFMA GEMM (chunked prefill)."""
    _f32(x, w, rank=2)
    check(x.shape[1] == w.shape[0], "inner dimensions differ")
    return _launch("gemm_auto_f32_gpu", [x, w], [(x.shape[0], w.shape[1])])


def gemm_auto_bias_gelu_f32_gpu(x, w, b):
    """gelu_tanh(x @ w + b): M = 1 -> GEMV with the fused epilogue, else the GEMM with it."""
    _f32(x, w, rank=2)
    check(x.shape[1] == w.shape[0] and tuple(b.shape) == (w.shape[1],), "shape mismatch")
    return _launch("gemm_auto_bias_gelu_f32_gpu", [x, w, b], [(x.shape[0], w.shape[1])])


def arange_offset_i64_gpu(pos, length):
    """(MI355X backend; the reference's arange_offset_i64_cpu on the device) i64[length] = pos[0] + [0 .. length-1]."""
    check(pos.dtype == i64 and tuple(pos.shape) == (1,), "pos must be i64[1]")
    return _launch("arange_offset_i64_gpu", [pos], [(int(length),)], dict(length=int(length)), out_dtypes=[i64])


# ---- Kokoro frame-rate (channel-last) -------------------------------------------------------------------------

def channel_stats_lc_f32_gpu(x):
    """Per-(128-row chunk, channel) (mean, M2) of x f32[L, C] -> f32[ceil(L / 128), C, 2]."""
    _f32(x, rank=2)
    return _launch("channel_stats_lc_f32_gpu", [x], [(-(-x.shape[0] // STAT_CHUNK), x.shape[1], 2)])


def adain_affine_lc_f32_gpu(stats, gb, length, eps=1e-5):
    """AdaIN affine f32[3, C] = (mean, (1 + g) / std, b) from channel_stats_lc over `length` rows; channels past
    len(gb) / 2 get (0, 0, 0) (reference ops/kokoro_gpu.py:104-118)."""
    _f32(stats, rank=3)
    _f32(gb, rank=1)
    c = stats.shape[1]
    check(gb.shape[0] % 2 == 0 and gb.shape[0] // 2 <= c, "gb must be f32[2 Creal] with Creal <= C")
    check(stats.shape[0] == -(-int(length) // STAT_CHUNK), "stats chunks don't match length")
    return _launch("adain_affine_lc_f32_gpu", [stats, gb], [(3, c)], dict(eps=float(eps), length=int(length)))


def snake_affine_lc_f32_gpu(x, affine, alpha):
    _f32(x, affine, rank=2)
    check(affine.shape == (3, x.shape[1]) and alpha.shape == (x.shape[1],), "affine f32[3, C], alpha f32[C]")
    return _launch("snake_affine_lc_f32_gpu", [x, affine, alpha], [x.shape])


def leaky_lc_f32_gpu(x, slope, affine=None):
    _f32(x, rank=2)
    if affine is None:
        return _launch("leaky_lc_f32_gpu", [x], [x.shape], dict(slope=float(slope)))
    check(affine.shape == (3, x.shape[1]), "affine must be f32[3, C]")
    return _launch("leaky_affine_lc_f32_gpu", [x, affine], [x.shape], dict(slope=float(slope)))


def convt_gather_lc_f32_gpu(y, b, kernel, stride, padding, add=None, reflect_left=False):
    """ConvTranspose1d overlap-add of y = x @ W[Ci, K*Co] (f32[Lin, K*Co]) + b [+ add] -> f32[Lout, Co]
    (reference ops/kokoro_gpu.py:151-160; `kernel` is the kernel size)."""
    k = int(kernel)
    _f32(y, rank=2)
    co = b.shape[0]
    check(y.shape[1] == k * co, "y must be f32[Lin, K * Co]")
    rl = 1 if reflect_left else 0
    lout = (y.shape[0] - 1) * stride - 2 * padding + k + rl
    check(lout >= (2 if rl else 1), "empty convT output")
    attrs = dict(kernel=k, padding=int(padding), reflect_left=rl, stride=int(stride))
    if add is None:
        return _launch("convt_gather_lc_f32_gpu", [y, b], [(lout, co)], attrs)
    check(tuple(add.shape) == (lout, co), "add shape mismatch")
    return _launch("convt_gather_add_lc_f32_gpu", [y, b, add], [(lout, co)], attrs)



def dwconvt_lc_f32_gpu(x, w, b, stride=2, padding=1):
    _f32(x, w, rank=2)
    check(w.shape[0] == x.shape[1] and b.shape == (x.shape[1],), "w must be f32[C, K], b f32[C]")
    lout = (x.shape[0] - 1) * stride - 2 * padding + w.shape[1] + (stride - 1)
    return _launch("dwconvt_lc_f32_gpu", [x, w, b], [(lout, x.shape[1])], dict(padding=int(padding), stride=int(stride)))


def upsample2_lc_f32_gpu(x):
    _f32(x, rank=2)
    return _launch("upsample2_lc_f32_gpu", [x], [(2 * x.shape[0], x.shape[1])])


def concat_pad_lc_f32_gpu(a, b=None, cout=None):
    _f32(a, rank=2)
    cb = 0 if b is None else b.shape[1]
    total = a.shape[1] + cb
    cout = -(-total // 16) * 16 if cout is None else int(cout)
    check(cout >= total, "cout smaller than the concatenation")
    if b is None:
        return _launch("pad_cols_lc_f32_gpu", [a], [(a.shape[0], cout)], dict(cout=cout))
    check(a.shape[0] == b.shape[0], "row counts differ")
    return _launch("concat_pad_lc_f32_gpu", [a, b], [(a.shape[0], cout)], dict(cout=cout))


def lc_to_cf_f32_gpu(x, channels):
    _f32(x, rank=2)
    check(x.shape[1] >= channels, "channels exceeds the padded width")
    return _launch("lc_to_cf_f32_gpu", [x], [(int(channels), x.shape[0])], dict(channels=int(channels)))


def transpose_f32_gpu(x):
    _f32(x, rank=2)
    return _launch("transpose_f32_gpu", [x], [(x.shape[1], x.shape[0])])


def add_f32_gpu(a, b):
    _f32(a, b)
    check(tuple(a.shape) == tuple(b.shape), "shape mismatch")
    return _launch("add_f32_gpu", [a, b], [a.shape])


def mul_f32_gpu(a, b):
    _f32(a, b)
    check(tuple(a.shape) == tuple(b.shape), "shape mismatch")
    return _launch("mul_f32_gpu", [a, b], [a.shape])


def add3_scale_f32_gpu(a, b, c, scale):
    _f32(a, b, c)
    check(tuple(a.shape) == tuple(b.shape) == tuple(c.shape), "add3 shape mismatch")
    return _launch("add3_scale_f32_gpu", [a, b, c], [a.shape], dict(scale=float(scale)))


def istft_logits_lc_f32_gpu(x, n_fft=20, hop=5):
    """torch.istft(exp(m) e^{i sin(p)}, periodic hann, center) from channel-last logits x f32[L, Cpad] -> f32[hop (L - 1)]
    (reference ops/kokoro_gpu.py:183-195)."""
    _f32(x, rank=2)
    check(n_fft >= 2 and n_fft % 2 == 0 and hop >= 1 and x.shape[1] >= n_fft + 2 and x.shape[0] >= 2, "bad iSTFT")
    return _launch("istft_logits_lc_f32_gpu", [x], [(hop * (x.shape[0] - 1),)], dict(hop=int(hop), n_fft=int(n_fft)))


# ---- token-rate front end (MI355X backend: the reference runs these on the host) ------------------------------

def embedding_f32_gpu(table, ids):
    """(MI355X backend) rows of table f32[V, D] at ids i64[N] -> f32[N, D]; an out-of-range id gives a NaN row
    (the reference's embedding_f32_cpu reports an error instead; a device kernel cannot)."""
    _f32(table, rank=2)
    check(ids.dtype == i64 and ids.ndim == 1, "ids must be i64[N]")
    return _launch("embedding_f32_gpu", [table, ids], [(ids.shape[0], table.shape[1])], out_dtypes=[f32])


def embedding2_add_f32_gpu(table, ids, table2, ids2):
    """(MI355X backend) table[ids] + table2[ids2] (GPT-2 token + position embedding) -> f32[N, D]."""
    _f32(table, table2, rank=2)
    check(table.shape[1] == table2.shape[1] and ids.shape == ids2.shape and ids.dtype == i64 == ids2.dtype,
          "embedding2_add: shape mismatch")
    return _launch("embedding2_add_f32_gpu", [table, ids, table2, ids2], [(ids.shape[0], table.shape[1])])


def argmax_f32_gpu(x):
    """(MI355X backend) first index of the row maximum of x f32[R, N] -> i64[R] (greedy decoding on device)."""
    _f32(x, rank=2)
    return _launch("argmax_f32_gpu", [x], [(x.shape[0],)], out_dtypes=[i64])


# ---- Kokoro token-rate sequence + signal kernels (MI355X backend: the reference runs these on the host) ------

def lstm_bidir_t_f32_gpu(x, w_ih, w_hh_t, b):
    """1-layer bidirectional nn.LSTM (gates i, f, g, o): x f32[T, I], w_ih f32[8H, I] (rows 0..4H forward),
    w_hh_t = W_hh^T f32[H, 8H], b = b_ih + b_hh f32[8H] -> f32[T, 2H] = [h_fwd | h_bwd]
    (reference lstm_bidir_t_f32_cpu, ops/kokoro.py:107-116)."""
    _f32(x, w_ih, w_hh_t, rank=2)
    h = w_hh_t.shape[0]
    check(w_ih.shape == (8 * h, x.shape[1]) and w_hh_t.shape[1] == 8 * h and tuple(b.shape) == (8 * h,),
          "expected w_ih [8H, I], w_hh_t [H, 8H], b [8H]")
    check(h <= 256, "H must be <= 256")
    return _launch("lstm_bidir_t_f32_gpu", [x, w_ih, w_hh_t, b], [(x.shape[0], 2 * h)])


def lstm2_bidir_t_f32_gpu(x1, w_ih1, w_hh_t1, b1, x2, w_ih2, w_hh_t2, b2):
    """(MI355X backend) Two lstm_bidir_t_f32_gpu of one length T and H = 256 in one recurrence launch:
    (f32[T, 2H], f32[T, 2H]), each equal to its own lstm_bidir_t_f32_gpu."""
    _f32(x1, w_ih1, w_hh_t1, x2, w_ih2, w_hh_t2, rank=2)
    h = w_hh_t1.shape[0]
    check(h == 256 and x1.shape[0] == x2.shape[0], "two LSTMs of one length with H = 256")
    for x, wi, wh, b in ((x1, w_ih1, w_hh_t1, b1), (x2, w_ih2, w_hh_t2, b2)):
        check(wi.shape == (8 * h, x.shape[1]) and tuple(wh.shape) == (h, 8 * h) and tuple(b.shape) == (8 * h,),
              "expected w_ih [8H, I], w_hh_t [H, 8H], b [8H]")
    t = x1.shape[0]
    return _launch("lstm2_bidir_t_f32_gpu", [x1, w_ih1, w_hh_t1, b1, x2, w_ih2, w_hh_t2, b2],
                   [(t, 2 * h), (t, 2 * h)])


def repeat_interleave_f32_gpu(x, dur, frames):
    """x.repeat_interleave(dur, 0) -> f32[frames, C]; dur is a device i64[T]. `frames` must equal sum(dur): the
    caller checks it on the host (reference repeat_interleave_f32_cpu reports a mismatch as an error)."""
    _f32(x, rank=2)
    check(dur.dtype == i64 and tuple(dur.shape) == (x.shape[0],), "dur must be i64[T]")
    check(x.shape[0] <= 8192, "T must be <= 8192")
    return _launch("repeat_interleave_f32_gpu", [x, dur], [(int(frames), x.shape[1])], dict(frames=int(frames)))


def adalayernorm_f32_gpu(x, gb, eps=1e-5):
    """(1 + gb[:C]) * LN_noaffine(x) + gb[C:] over x f32[R, C] (reference adalayernorm_f32_cpu, ops/kokoro.py:69)."""
    _f32(x, rank=2)
    check(tuple(gb.shape) == (2 * x.shape[1],) and x.shape[1] <= 2048, "gb must be f32[2C], C <= 2048")
    return _launch("adalayernorm_f32_gpu", [x, gb], [x.shape], dict(eps=float(eps)))


def concat_bcast_f32_gpu(x, v):
    """[x | v] per row: concat_cols(x, broadcast_rows(v)) for x f32[R, C1], v f32[C2] -> f32[R, C1 + C2]."""
    _f32(x, rank=2)
    _f32(v, rank=1)
    return _launch("concat_bcast_f32_gpu", [x, v], [(x.shape[0], x.shape[1] + v.shape[0])])


def harmonic_source_f32_gpu(f0, noise, w, b):
    """hn-NSF harmonic source with explicit SineGen noise: f0 f32[n], noise f32[300 n, 9], l_linear w f32[9],
    b f32[1] -> f32[300 n] (reference harmonic_source_f32_cpu, kernels/cpu/kokoro_signal.cpp:89-192)."""
    _f32(f0, w, b, rank=1)
    n = f0.shape[0]
    check(noise.shape == (300 * n, 9) and w.shape == (9,) and b.shape == (1,), "bad harmonic source operands")
    return _launch("harmonic_source_f32_gpu", [f0, noise, w, b], [(300 * n,)])


def stft_magphase_lc_f32_gpu(x, n_fft=20, hop=5, cpad=32):
    """torch.stft (periodic Hann, center, reflect) -> channel-last f32[S / hop + 1, cpad]: magnitude in columns
    0..K-1, phase in K..2K-1 (K = n_fft / 2 + 1), zero padding after (reference stft_magphase_f32_cpu, which
    returns the channel-first [2K, frames])."""
    _f32(x, rank=1)
    check(cpad >= n_fft + 2 and x.shape[0] > n_fft // 2, "bad STFT configuration")
    return _launch("stft_magphase_lc_f32_gpu", [x], [(x.shape[0] // hop + 1, int(cpad))],
                   dict(hop=int(hop), n_fft=int(n_fft)))


def conv1d_1ch_f32_gpu(x, w, b, stride=1, padding=0, out=None):
    """Single-channel conv1d: x f32[L], w f32[K], b f32[1] -> f32[Lo] (the decoder's F0_conv / N_conv); `out`
    optionally names a preallocated f32[Lo] destination (e.g. a row of a [2, Lo] buffer)."""
    _f32(x, w, b, rank=1)
    lo = (x.shape[0] + 2 * padding - w.shape[0]) // stride + 1
    check(lo >= 1, "empty conv output")
    if out is not None:
        check(out.dtype == f32 and tuple(out.shape) == (lo,), "out must be f32[Lo]")
    return _launch("conv1d_1ch_f32_gpu", [x, w, b], [(lo,)], dict(padding=int(padding), stride=int(stride)),
                   outs=None if out is None else [out])
