"""Winograd conv family on the GPU (wino_tf* -> wino_mm* -> wino_adain_affine) vs the float64 direct conv of the
oracle, over the reference's test shapes (tests/kernels/test_winograd_gpu.py:40-175 in lariaus/lokinfer) plus the
Kokoro generator's: conv 1e-4, snake / leaky fused 2e-4, stats mean 1e-5 and inverse std 1e-4."""
import math

import numpy as np
import pytest

from lokinfer_amd import winograd as W
from oracle import kernels as K

pytestmark = pytest.mark.gpu


def G(lk, a):
    return lk.from_numpy(np.ascontiguousarray(a, np.float32), device="gpu", copy=True)


def close(got, ref, tol):
    got = got.numpy() if hasattr(got, "numpy") else np.asarray(got)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got.astype(np.float64) - ref)
    bound = tol + tol * np.abs(ref)
    assert (err <= bound).all(), f"max excess {np.max(err - bound):.3e}"


def _pad(k, d):
    return d * (k // 2) if k % 2 == 0 else d * (k - 1) // 2


def _case(seed, l, ci, co, k):
    r = np.random.default_rng(seed)
    x = r.standard_normal((l, ci)).astype(np.float32)
    w = (r.standard_normal((co, ci, k)) / math.sqrt(ci * k)).astype(np.float32)
    b = r.standard_normal(co).astype(np.float32)
    return r, x, w, b


def _direct(h, w, b, pad, d, res=None, scale=1.0):
    # oracle conv takes w [Co, K, Ci]
    return K.conv1d_lc(h, np.transpose(w, (0, 2, 1)), b, padding=pad, dilation=d, residual=res, out_scale=scale)


CONVS = [(128, 128, 1000, 11, 5), (128, 128, 777, 7, 3), (256, 256, 300, 3, 1), (128, 128, 1001, 3, 5),
         (256, 256, 513, 7, 1), (128, 128, 37, 11, 3), (16, 64, 5, 3, 1), (128, 64, 1001, 7, 1),
         (32, 128, 70, 5, 2), (64, 64, 9, 12, 1), (16, 64, 40, 4, 1), (128, 128, 2, 3, 1),
         (256, 256, 1770, 3, 3), (128, 128, 10621, 11, 5),
         # one tap group with 48- and 32-channel pipeline steps (Ci / 16 divisible by 3, by 2)
         (144, 64, 500, 3, 1), (48, 128, 301, 3, 2), (96, 64, 257, 3, 1)]


@pytest.mark.parametrize("ci,co,l,k,d", CONVS)
@pytest.mark.parametrize("res", [False, True])
def test_wino_conv1d(gpu, ci, co, l, k, d, res):
    lk = gpu
    r, x, w, b = _case(ci + l + k + d, l, ci, co, k)
    pad = _pad(k, d)
    u, tr = W.wino_weights(w)
    if res:
        rr = r.standard_normal((l + 2 * pad - d * (k - 1), co)).astype(np.float32)
        ref = _direct(x, w, b, pad, d, rr, 0.5)
        got = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), k, residual=G(lk, rr),
                                            out_scale=0.5, padding=pad, dilation=d)
    else:
        ref = _direct(x, w, b, pad, d)
        got = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), k, padding=pad, dilation=d)
    close(got, ref, 1e-4)


def _affine(r, ci):
    return np.stack([r.standard_normal(ci) * 0.5, r.uniform(0.5, 1.5, ci), r.standard_normal(ci) * 0.3]).astype(
        np.float32)


@pytest.mark.parametrize("ci,co,l,k,d", [(128, 128, 1000, 11, 5), (256, 256, 300, 3, 3), (128, 128, 501, 7, 1)])
def test_wino_conv1d_snake(gpu, ci, co, l, k, d):
    lk = gpu
    r, x, w, b = _case(l + k, l, ci, co, k)
    x = x * 2
    af, alpha = _affine(r, ci), r.uniform(0.2, 3.0, ci).astype(np.float32)
    pad = _pad(k, d)
    ref = _direct(K.affine_act(x, af, alpha, "snake"), w, b, pad, d)
    u, tr = W.wino_weights(w)
    got = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), k, padding=pad, dilation=d,
                                        affine=G(lk, af), alpha=G(lk, alpha))
    close(got, ref, 2e-4)


@pytest.mark.parametrize("ci,co,l", [(1104, 1024, 147), (528, 1024, 60), (256, 256, 294)])
@pytest.mark.parametrize("res", [False, True])
def test_wino_conv1d_leaky(gpu, ci, co, l, res):
    lk = gpu
    r, x, w, b = _case(l + ci, l, ci, co, 3)
    x = x * 2
    af = _affine(r, ci)
    h = K.affine_act(x, af, None, "leaky", 0.2)
    u, tr = W.wino_weights(w)
    kw, rr = {}, None
    if res:
        rr = r.standard_normal((l, co)).astype(np.float32)
        kw = dict(residual=G(lk, rr), out_scale=0.7071)
    ref = _direct(h, w, b, 1, 1, rr, 0.7071 if res else 1.0)
    got = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), 3, padding=1, affine=G(lk, af),
                                        slope=0.2, **kw)
    close(got, ref, 2e-4)


def _check_affine(af, y, gb, co):
    y64 = y.astype(np.float64)
    mean, var = y64.mean(0), y64.var(0)
    np.testing.assert_allclose(af[0], mean, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(af[1], (1 + gb[:co]) / np.sqrt(var + 1e-5), rtol=1e-4)
    assert np.array_equal(af[2], gb[co:])


@pytest.mark.parametrize("ci,co,l,k,d", [(128, 128, 1000, 11, 5), (128, 128, 777, 7, 3), (256, 256, 300, 3, 1),
                                         (128, 128, 129, 3, 1), (128, 64, 5, 7, 3), (64, 64, 300, 12, 2),
                                         (256, 256, 700, 7, 3), (256, 128, 300, 11, 5)])  # split-K, dilated stats
@pytest.mark.parametrize("res", [False, True])
def test_wino_stats_epilogue_affine(gpu, ci, co, l, k, d, res):
    lk = gpu
    r, x, w, b = _case(l + k + d, l, ci, co, k)
    b = b + 3  # a non-zero mean
    gb = (r.standard_normal(2 * co) * 0.3).astype(np.float32)
    pad = _pad(k, d)
    lo = l + 2 * pad - d * (k - 1)  # even K: one row longer per dilation
    u, tr = W.wino_weights(w)
    kw, rr = {}, None
    if res:
        rr = r.standard_normal((lo, co)).astype(np.float32)
        kw = dict(residual=G(lk, rr), out_scale=0.5)
    y, st = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), k, padding=pad, dilation=d,
                                          stats=True, **kw)
    assert st.shape == (W.stats_chunks(lo, d) * d, co, 2)
    close(y, _direct(x, w, b, pad, d, rr, 0.5 if res else 1.0), 1e-4)
    yn = y.numpy()
    if d == 1:  # the statistics layout equals channel_stats_lc's for d = 1
        np.testing.assert_allclose(st.numpy(), K.channel_stats_lc(yn), rtol=1e-4, atol=1e-4)
    af = lk.ops.wino_adain_affine_lc_f32_gpu(st, G(lk, gb), lo, dilation=d).numpy()
    _check_affine(af, yn, gb, co)


def test_wino_affine_padded_channels(gpu):
    """Creal < C: channels past Creal get an all-zero affine (the decoder's padded widths)."""
    lk = gpu
    r, x, w, b = _case(5, 300, 128, 128, 3)
    u, tr = W.wino_weights(w)
    y, st = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), 3, padding=1, stats=True)
    gb = (r.standard_normal(2 * 100) * 0.3).astype(np.float32)
    af = lk.ops.wino_adain_affine_lc_f32_gpu(st, G(lk, gb), 300).numpy()
    assert not af[:, 100:].any()
    y64 = y.numpy().astype(np.float64)[:, :100]
    np.testing.assert_allclose(af[0, :100], y64.mean(0), atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(af[1, :100], (1 + gb[:100]) / np.sqrt(y64.var(0) + 1e-5), rtol=1e-4)
    assert np.array_equal(af[2, :100], gb[100:])


@pytest.mark.parametrize("ci,co,l,d", [(256, 256, 300, 1), (128, 128, 1001, 5), (16, 64, 5, 1), (128, 128, 4097, 3)])
@pytest.mark.parametrize("stats", [False, True])
def test_wino_f23(gpu, ci, co, l, d, stats):
    lk = gpu
    r, x, w, b = _case(ci + l + d, l, ci, co, 3)
    rr = r.standard_normal((l, co)).astype(np.float32)
    ref = _direct(x, w, b, d, d, rr, 0.5)
    u, tr = W.wino_weights(w, tile=2)
    assert u.shape[0] == 4
    out = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), 3, residual=G(lk, rr), out_scale=0.5,
                                        padding=d, dilation=d, stats=stats)
    if stats:
        out, st = out
        af = lk.ops.wino_adain_affine_lc_f32_gpu(st, G(lk, np.zeros(2 * co, np.float32)), l, dilation=d).numpy()
        np.testing.assert_allclose(af[0], out.numpy().astype(np.float64).mean(0), atol=1e-5, rtol=1e-5)
    close(out, ref, 1e-4)


def test_wino_split_ops_and_rejects(gpu):
    """The two-launch pair called op by op equals conv1d_wino; bad operands raise before any launch."""
    lk = gpu
    r, x, w, b = _case(11, 200, 64, 64, 7)
    u, tr = W.wino_weights(w)
    attrs = dict(dilation=3, groups=2, kernel=7, padding=9, tile=4)
    v = lk.ops.wino_tf_lc_f32_gpu(G(lk, x), G(lk, tr), **attrs)
    assert v.shape == (W.tiles_rows(200, 3, 2, 4, 7), 64)
    y = lk.ops.wino_mm_lc_f32_gpu(v, G(lk, u), G(lk, b), G(lk, tr), G(lk, x), **attrs)
    y2 = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), 7, padding=9, dilation=3)
    assert np.array_equal(y.numpy(), y2.numpy())
    with pytest.raises(ValueError):  # Ci not a multiple of 16
        lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x[:, :40]), G(lk, u), G(lk, b), G(lk, tr), 7, padding=9, dilation=3)
    with pytest.raises(ValueError):  # padding not a multiple of the dilation
        lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), 7, padding=8, dilation=3)
    with pytest.raises(ValueError):  # U for another kernel size
        lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), 3, padding=3, dilation=3)


def _mm_workgroups(lo, co, d, tile):
    """Workgroups of one wino_mm launch (csrc/winograd.hip lk_hip_wino_mm_lc_f32, no split): 64 output channels x
    64 tiles of one residue class each. Above 512 (two per CU) the three-per-CU instantiations run."""
    tiles = -(-(-(-lo // d)) // tile)
    return (co // 64) * (-(-tiles // 64)) * d


# Grids above 512 workgroups: the only shapes that select winoMmKernel<4,6,1,3>, <4,7,2,3> and <4,7,3,3> (the
# Kokoro-487 generator's convs). Each runs with the fused affine + Snake, the residual and the stats epilogue,
# as the generator's resblocks do.
LARGE = [(128, 128, 80000, 11, 5), (256, 256, 48880, 7, 3), (128, 128, 70000, 3, 1), (128, 128, 80000, 3, 5)]


@pytest.mark.parametrize("ci,co,l,k,d", LARGE)
def test_wino_large_grid_instantiations(gpu, ci, co, l, k, d):
    lk = gpu
    r, x, w, b = _case(l + 3 * k + d, l, ci, co, k)
    pad = _pad(k, d)
    assert _mm_workgroups(l, co, d, 4) > 512
    af, alpha = _affine(r, ci), r.uniform(0.2, 3.0, ci).astype(np.float32)
    rr = r.standard_normal((l, co)).astype(np.float32)
    u, tr = W.wino_weights(w)
    y, st = lk.ops.conv1d_wino_lc_f32_gpu(G(lk, x), G(lk, u), G(lk, b), G(lk, tr), k, residual=G(lk, rr),
                                          padding=pad, dilation=d, affine=G(lk, af), alpha=G(lk, alpha), stats=True)
    ref = _direct(K.affine_act(x, af, alpha, "snake"), w, b, pad, d, rr)
    close(y, ref, 2e-4)
    yn = y.numpy()
    assert st.shape == (W.stats_chunks(l, d) * d, co, 2)
    if d == 1:
        np.testing.assert_allclose(st.numpy(), K.channel_stats_lc(yn), rtol=1e-4, atol=1e-4)
    gb = (r.standard_normal(2 * co) * 0.3).astype(np.float32)
    af2 = lk.ops.wino_adain_affine_lc_f32_gpu(st, G(lk, gb), l, dilation=d).numpy()
    _check_affine(af2, yn, gb, co)


@pytest.mark.parametrize("ci,co,l,k,d", CONVS[:10] + [(1104, 1024, 300, 3, 1), (144, 64, 500, 3, 1)] + LARGE[:2])
def test_wino_u_layouts_agree(gpu, ci, co, l, k, d):
    """u_layout 1 (U transposed, the Kokoro graph's form) runs the same MFMAs in the same order as the reference
    layout: the outputs and statistics are the same bits (small grids through the split-K path too)."""
    lk = gpu
    r, x, w, b = _case(ci + 2 * l + k, l, ci, co, k)
    pad = _pad(k, d)
    u, tr = W.wino_weights(w)
    ut, tr2 = W.wino_weights_t(w)
    n = W.variant(k)[1]
    # the tiled element (x, cb, c, g, k4, j, q) is U[x, g Ci + 16 c + 4 k4 + q, 64 cb + j]
    t = ut.reshape(u.shape[0], co // 64, ci // 16, n, 4, 64, 4)
    x_, cb, c, g, k4, j, q = 1, co // 64 - 1, ci // 16 - 1, n - 1, 2, 37, 3
    assert t[x_, cb, c, g, k4, j, q] == u[x_, g * ci + 16 * c + 4 * k4 + q, 64 * cb + j]
    assert np.array_equal(tr, tr2) and np.array_equal(np.sort(ut.ravel()), np.sort(u.ravel()))
    args = (G(lk, x), None, G(lk, b), G(lk, tr), k)
    y0, s0 = lk.ops.conv1d_wino_lc_f32_gpu(args[0], G(lk, u), *args[2:], padding=pad, dilation=d, stats=True)
    y1, s1 = lk.ops.conv1d_wino_lc_f32_gpu(args[0], G(lk, ut), *args[2:], padding=pad, dilation=d, stats=True,
                                           u_layout=1)
    assert np.array_equal(y0.numpy(), y1.numpy())
    assert np.array_equal(s0.numpy(), s1.numpy())
