"""GPU parity of the f16 op family (lk.ops.f16_gpu) against the float64 composition of the contract
(oracle/qwen3.py, inputs drawn as f16; the contract's intermediate roundings kept, the output's own rounding left
out), with the reference's tolerance construction
(tests/kernels/test_f16_basic_gpu.py:7-28, test_f16_fused_gpu.py in lariaus/lokinfer): one f16 rounding of the exact
result (U = 2^-11 relative, + half the subnormal spacing) plus an op-specific float32 term:
  GEMM / LM head   2^-22 sqrt(K) * sqrt(sum_k (x_k w_k)^2)
  rmsnorm          2^-10 |g h| (the float h may round to the other f16 neighbour than the float64 h)
  rope             2^-20 (|x_j| + |x_j+64|)
  attention        2^-22 (8 + sqrt(P)) max|v|  (f32 softmax; P.V with P in two f16 parts, ~22 bits)
  elementwise      2^-20 |ref|
Fused ops are also checked bit for bit against the composition of this backend's own basic ops where the backend
promises it (the M = 1 rmsnorm GEMV and the QK-norm share the row kernel's sum order). Shapes: Qwen3's (K = 2048,
6144; N = 4096, 12288; 16 / 8 heads; caches to 2048 rows) and odd sizes, M = 1 and prefill M (44, 401, 416)."""
import numpy as np
import pytest
import torch

from lokinfer_amd._lib import LokinferError, check_device_errors

from oracle import qwen3 as Q

pytestmark = pytest.mark.gpu

U, SUB = 2.0 ** -11, 2.0 ** -25
O = Q.Ops(np.float64)                   # the contract's intermediate roundings
X = Q.Ops(np.float64, rounding=False)   # exact final results: the tolerance prices their one rounding
rng = np.random.default_rng(99)


def h16(*shape, scale=1.0):
    return (scale * rng.standard_normal(shape)).astype(np.float16)


def G(lk, a):
    return lk.from_numpy(np.ascontiguousarray(a), device="gpu", copy=True)


def P(lk, p):
    return G(lk, np.array([p], np.int64))


def check(got, ref, extra=0.0, what=""):
    got = np.asarray(got.numpy() if hasattr(got, "numpy") else got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.isfinite(got).all(), f"{what}: non-finite output"
    tol = U * (1 + 2.0 ** -10) * np.abs(ref) + extra + SUB
    err = np.abs(got - ref)
    bad = err > tol
    if bad.any():
        i = np.unravel_index(np.argmax(err - tol), err.shape)
        raise AssertionError(f"{what}: {bad.sum()} / {bad.size} beyond tolerance; worst at {i}: got {got[i]!r} "
                             f"ref {ref[i]!r} err {err[i]:.3g} tol {np.broadcast_to(tol, err.shape)[i]:.3g}")


def gemm_term(x, w):
    x, w = np.asarray(x, np.float64), np.asarray(w, np.float64)
    return 2.0 ** -22 * np.sqrt(x.shape[1]) * np.sqrt((x * x) @ (w * w))


@pytest.mark.parametrize("m,k,n", [(1, 2048, 4096), (44, 2048, 2048), (401, 2048, 1024), (416, 6144, 2048),
                                   (3, 40, 24), (70, 200, 130), (1, 6144, 2048), (128, 2048, 4096),
                                   # the 128-row tile (M >= 1024): split-K grid, K tail with ragged M and N, full grid
                                   (1024, 2048, 1024), (1100, 200, 300), (1024, 2048, 4096)])
def test_gemm(gpu, m, k, n):
    lk = gpu
    F = lk.ops.f16_gpu
    x, w = h16(m, k), h16(k, n, scale=1 / np.sqrt(k))
    pw = F.pack(w)
    ref, ft = X.gemm(x, w), gemm_term(x, w)
    check(F.gemm_opt_f16_gpu(G(lk, x), pw), ref, ft, "gemm_opt")
    check(F.gemm_f16_gpu(G(lk, x), G(lk, w)), ref, ft, "gemm (raw weight, packed per call)")
    res, b = h16(m, n), h16(n)
    check(F.gemm_add_opt_f16_gpu(G(lk, x), pw, G(lk, res)), O.c(res) + O.c(x) @ O.c(w),
          ft + 2.0 ** -23 * np.abs(O.c(res) + O.c(x) @ O.c(w)), "gemm_add_opt")
    check(F.gemm_bias_opt_f16_gpu(G(lk, x), pw, G(lk, b)), O.c(x) @ O.c(w) + O.c(b),
          ft + 2.0 ** -23 * np.abs(O.c(x) @ O.c(w) + O.c(b)), "gemm_bias_opt")


# M >= 256 runs the 128-row tile: (416, 2048, 6144) on a full grid, (300, 520, 200) with a K tail and ragged M and
# N, (512, 2048, 512) split over K
@pytest.mark.parametrize("m,k,n", [(1, 2048, 6144), (44, 2048, 6144), (416, 2048, 6144), (5, 64, 40),
                                   (300, 520, 200), (512, 2048, 512)])
def test_gemm_swiglu(gpu, m, k, n):
    lk = gpu
    F = lk.ops.f16_gpu
    x, wg, wu = h16(m, k), h16(k, n, scale=1 / np.sqrt(k)), h16(k, n, scale=1 / np.sqrt(k))
    g, u = O.c(x) @ O.c(wg), O.c(x) @ O.c(wu)
    sg = np.abs(g / (1 + np.exp(-g)))
    ref = g / (1 + np.exp(-g)) * u
    tol = 1.1 * np.abs(u) * gemm_term(x, wg) + sg * gemm_term(x, wu) + 2.0 ** -20 * np.abs(ref)
    check(F.gemm_swiglu_opt_f16_gpu(G(lk, x), F.pack(np.concatenate([wg, wu], 1))), ref, tol, "gemm_swiglu_opt")


@pytest.mark.parametrize("m", [1, 7, 416])
@pytest.mark.parametrize("swiglu", [False, True])
def test_rmsnorm_gemm(gpu, m, swiglu):
    lk = gpu
    F = lk.ops.f16_gpu
    k, n = 2048, 1024
    x, g = h16(m, k, scale=3.0), (1 + 0.1 * rng.standard_normal(k)).astype(np.float16)
    w = h16(k, 2 * n if swiglu else n, scale=1 / np.sqrt(k))
    pw = F.pack(w)
    X, Gm = G(lk, x), G(lk, g)
    a = F.rmsnorm_f16_gpu(X, Gm)
    h = O.r16(O.c(x) / np.sqrt((O.c(x) ** 2).mean(-1, keepdims=True) + 1e-6))
    check(a, O.c(g) * h, 2.0 ** -10 * np.abs(O.c(g) * h), "rmsnorm")
    if swiglu:
        y, _ = F.rmsnorm_gemm_swiglu_opt_f16_gpu(X, Gm, pw)
        comp = F.gemm_swiglu_opt_f16_gpu(a, pw)
    else:
        y, _ = F.rmsnorm_gemm_opt_f16_gpu(X, Gm, pw)
        comp = F.gemm_opt_f16_gpu(a, pw)
    # the fused op equals this backend's composition bit for bit (the GEMV normalizes with the row kernel's order)
    np.testing.assert_array_equal(y.numpy().view(np.uint16), comp.numpy().view(np.uint16))


@pytest.mark.parametrize("t,d,v", [(1, 2048, 151936), (416, 2048, 151936), (3, 64, 1001)])
def test_lm_head_last(gpu, t, d, v):
    lk = gpu
    F = lk.ops.f16_gpu
    x, tab = h16(t, d), h16(v, d, scale=0.02)
    ref = O.c(x[-1:]) @ O.c(tab).T
    tol = 2.0 ** -22 * np.sqrt(d) * np.sqrt((O.c(x[-1:]) ** 2) @ (O.c(tab) ** 2).T) + 2.0 ** -23 * np.abs(ref)
    for op in (F.lm_head_last_f16_gpu, F.lm_head_last_opt_f16_gpu):
        got = op(G(lk, x), G(lk, tab)).numpy()
        assert got.dtype == np.float32 and got.shape == (1, v)
        err = np.abs(got - ref)
        assert (err <= tol + 1e-30).all(), err.max()


@pytest.mark.parametrize("t,pos", [(1, 0), (1, 1999), (44, 0), (401, 13), (5, 100000)])
def test_rmsnorm_heads_rope_qknorm(gpu, t, pos):
    lk = gpu
    F = lk.ops.f16_gpu
    qh, kvh, cap = 16, 8, max(2048, pos + t)
    qkv = h16(t, 128 * (qh + 2 * kvh), scale=2.0)
    qg, kg = (1 + 0.1 * rng.standard_normal(128)).astype(np.float16), (1 + 0.1 * rng.standard_normal(128)).astype(np.float16)
    Qkv, Pp = G(lk, qkv), P(lk, pos)
    dq, dk = 128 * qh, 128 * kvh
    for sl, g in ((slice(0, dq), qg), (slice(dq, dq + dk), kg)):
        x = np.ascontiguousarray(qkv[:, sl])
        n = F.rmsnorm_heads_f16_gpu(G(lk, x), G(lk, g))
        xh = O.c(x).reshape(t, -1, 128)
        hh = O.r16(xh / np.sqrt((xh ** 2).mean(-1, keepdims=True) + 1e-6)).reshape(t, -1)
        gh = O.c(np.tile(g, x.shape[1] // 128)) * hh
        check(n, gh, 2.0 ** -10 * np.abs(gh), "rmsnorm_heads")
        nn = n.numpy()
        r = F.rope_f16_gpu(n, Pp)
        lo, hi = O.c(nn).reshape(t, -1, 2, 64)[:, :, 0], O.c(nn).reshape(t, -1, 2, 64)[:, :, 1]
        extra = 2.0 ** -20 * np.repeat((np.abs(lo) + np.abs(hi))[:, :, None, :], 2, 2).reshape(t, -1)
        check(r, X.rope(nn, pos), extra, "rope")
    kc, vc = G(lk, np.zeros((cap, dk), np.float16)), G(lk, np.zeros((cap, dk), np.float16))
    q = F.qknorm_rope_kv_opt_f16_gpu(Qkv, G(lk, qg), G(lk, kg), Pp, kc, vc)
    # bit for bit against the composition of the basic ops
    qb = F.rope_f16_gpu(F.rmsnorm_heads_f16_gpu(G(lk, np.ascontiguousarray(qkv[:, :dq])), G(lk, qg)), Pp)
    kb = F.rope_f16_gpu(F.rmsnorm_heads_f16_gpu(G(lk, np.ascontiguousarray(qkv[:, dq:dq + dk])), G(lk, kg)), Pp)
    np.testing.assert_array_equal(q.numpy().view(np.uint16), qb.numpy().view(np.uint16))
    np.testing.assert_array_equal(kc.numpy()[pos:pos + t].view(np.uint16), kb.numpy().view(np.uint16))
    np.testing.assert_array_equal(vc.numpy()[pos:pos + t].view(np.uint16), qkv[:, dq + dk:].view(np.uint16))
    assert not kc.numpy()[:pos].any() and not kc.numpy()[pos + t:].any()


def _attn_case(t, pos, qh, kvh, cap):
    q = h16(t, 128 * qh)
    kc, vc = h16(cap, 128 * kvh), h16(cap, 128 * kvh)
    return q, kc, vc


# caches of 128 chunks or more take two q heads per wave; past 128 chunks (cap 20000: 313) a wave runs 3
# consecutive chunks
@pytest.mark.parametrize("t,pos,cap", [(1, 0, 64), (1, 415, 480), (1, 1999, 2048), (1, 64, 2048), (2, 0, 64),
                                       (44, 0, 480), (416, 0, 480), (33, 100, 480), (70, 7, 300), (300, 1500, 2048),
                                       (1, 70, 20000), (1, 9000, 20000), (1, 19999, 20000)])
def test_attention_gqa(gpu, t, pos, cap):
    lk = gpu
    F = lk.ops.f16_gpu
    qh, kvh = 16, 8
    q, kc, vc = _attn_case(t, pos, qh, kvh, cap)
    ref = X.attention_gqa(q, kc, vc, pos, qh, kvh)
    extra = 2.0 ** -22 * (8 + np.sqrt(pos + t)) * np.abs(O.c(vc[:pos + t])).max()
    for op in (F.attention_gqa_f16_gpu, F.attention_gqa_opt_f16_gpu):
        got = op(G(lk, q), G(lk, kc), G(lk, vc), P(lk, pos), q_heads=qh, kv_heads=kvh)
        check(got, ref, extra, f"attention_gqa t={t} pos={pos}")


def test_attention_gqa_small_group_counts(gpu):
    lk = gpu
    F = lk.ops.f16_gpu
    for qh, kvh in ((2, 2), (4, 1), (8, 2)):
        for t, pos in ((1, 70), (37, 5)):
            q, kc, vc = _attn_case(t, pos, qh, kvh, 128)
            got = F.attention_gqa_opt_f16_gpu(G(lk, q), G(lk, kc), G(lk, vc), P(lk, pos), q_heads=qh, kv_heads=kvh)
            extra = 2.0 ** -22 * (8 + np.sqrt(pos + t)) * np.abs(O.c(vc[:pos + t])).max()
            check(got, X.attention_gqa(q, kc, vc, pos, qh, kvh), extra, f"gqa {qh}/{kvh} t={t}")


def test_rows_past_the_cache(gpu):
    lk = gpu
    F = lk.ops.f16_gpu
    cap, pos, t = 64, 60, 8
    k, v = h16(t, 1024), h16(t, 1024)
    kc, vc = G(lk, np.zeros((cap, 1024), np.float16)), G(lk, np.zeros((cap, 1024), np.float16))
    F.kv_write_f16_gpu(kc, vc, G(lk, k), G(lk, v), P(lk, pos))
    check_device_errors()  # the cache write drops the rows past the end without recording an error
    np.testing.assert_array_equal(kc.numpy()[pos:], k[:cap - pos])
    np.testing.assert_array_equal(vc.numpy()[pos:], v[:cap - pos])
    assert not kc.numpy()[:pos].any()
    q = h16(t, 2048)
    out = F.attention_gqa_opt_f16_gpu(G(lk, q), kc, vc, P(lk, pos))
    with pytest.raises(LokinferError, match="device error 2.*detail 64"):  # the first query without a cache row
        check_device_errors()
    got = out.numpy().astype(np.float64)
    ref = X.attention_gqa(q[:cap - pos], kc.numpy(), vc.numpy(), pos, 16, 8)
    check(got[:cap - pos], ref, 2.0 ** -22 * (8 + 8) * np.abs(v).max(), "fitting rows")
    assert np.isnan(got[cap - pos:]).all()


def test_embedding_scatter_elementwise(gpu):
    lk = gpu
    F = lk.ops.f16_gpu
    tab = h16(151936, 64)
    ids = rng.integers(0, 151936, 50)
    ids[[3, 4, 10, 49]] = Q.PAD_ID
    audio = h16(4, 64)
    I = G(lk, ids.astype(np.int64))
    e = F.embedding_f16_gpu(I, G(lk, tab))
    np.testing.assert_array_equal(e.numpy(), tab[ids])
    s = F.scatter_audio_f16_gpu(e, I, G(lk, audio)).numpy()
    np.testing.assert_array_equal(s, O.scatter_audio(tab[ids], ids, audio).astype(np.float16))
    s3 = F.scatter_audio_f16_gpu(e, I, G(lk, audio[:3]))  # a pad row without an audio row: NaN, and recorded
    with pytest.raises(LokinferError, match="device error 5.*detail 49"):
        check_device_errors()
    s3 = s3.numpy()
    assert np.isnan(s3[49]).all() and np.array_equal(s3[:49], s[:49])
    bad = F.embedding_f16_gpu(G(lk, np.array([5, -1, 151936], np.int64)), G(lk, tab))
    with pytest.raises(LokinferError, match="device error 3"):
        check_device_errors()
    bad = bad.numpy()
    assert np.array_equal(bad[0], tab[5]) and np.isnan(bad[1:]).all()
    a, b = h16(33, 70, scale=4.0), h16(33, 70, scale=4.0)
    check(F.add_f16_gpu(G(lk, a), G(lk, b)), X.add(a, b), 2.0 ** -20 * np.abs(O.c(a) + O.c(b)), "add")
    sm = X.silu_mul(a, b)
    check(F.silu_mul_f16_gpu(G(lk, a), G(lk, b)), sm, 2.0 ** -20 * np.abs(sm) + 2.0 ** -24, "silu_mul")


@pytest.mark.parametrize("pos,cap", [(0, 64), (63, 480), (64, 480), (200, 300), (415, 480), (511, 512), (1000, 1024),
                                     (1999, 2048),
                                     (5000, 8192), (8300, 20000), (19999, 20000)])
def test_decode_fusions_equal_compositions(gpu, pos, cap):
    """The decode-step fusions give the bits of the ops they replace: attention_decode_qkr vs qknorm_rope_kv +
    attention_gqa (output and both caches), twice in a row with the same counters (each call leaves them zero);
    rmsnorm_lm_head_last vs rmsnorm + lm_head_last."""
    lk = gpu
    F = lk.ops.f16_gpu
    qh, kvh = 16, 8
    counters = lk.from_numpy(np.zeros(qh, np.int32), device="gpu", copy=True)
    for rep in range(2):
        qkv = h16(1, 128 * (qh + 2 * kvh), scale=2.0)
        qg = (1 + 0.1 * rng.standard_normal(128)).astype(np.float16)
        kg = (1 + 0.1 * rng.standard_normal(128)).astype(np.float16)
        kc0, vc0 = h16(cap, 1024), h16(cap, 1024)
        p = pos - rep
        Pp = P(lk, p)
        ka, va, kb, vb = G(lk, kc0), G(lk, vc0), G(lk, kc0), G(lk, vc0)
        q = F.qknorm_rope_kv_opt_f16_gpu(G(lk, qkv), G(lk, qg), G(lk, kg), Pp, ka, va)
        ref = F.attention_gqa_opt_f16_gpu(q, ka, va, Pp)
        got = F.attention_decode_qkr_opt_f16_gpu(G(lk, qkv), G(lk, qg), G(lk, kg), Pp, kb, vb, counters)
        if p < 0:  # an invalid position: NaN outputs and no cache write on both sides, recorded on the device
            with pytest.raises(LokinferError, match="device error 2.*detail -1"):
                check_device_errors()
        ref, got = ref.numpy(), got.numpy()
        np.testing.assert_array_equal(got.view(np.uint16), ref.view(np.uint16))
        np.testing.assert_array_equal(kb.numpy().view(np.uint16), ka.numpy().view(np.uint16))
        np.testing.assert_array_equal(vb.numpy().view(np.uint16), va.numpy().view(np.uint16))
        assert not counters.numpy().any()
    x, g, tab = h16(3, 2048), (1 + 0.1 * rng.standard_normal(2048)).astype(np.float16), h16(5000, 2048, scale=0.02)
    a = F.lm_head_last_opt_f16_gpu(F.rmsnorm_f16_gpu(G(lk, x), G(lk, g)), G(lk, tab)).numpy()
    b = F.rmsnorm_lm_head_last_opt_f16_gpu(G(lk, x), G(lk, g), G(lk, tab)).numpy()
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
