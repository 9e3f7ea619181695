"""GPU parity of the chunked-generate ops (kv_write_rows, attention_cache / attention_gen, split-K partials and their
bias + residual + LayerNorm consumer, gemm_auto, arange_offset) against the numpy oracle (oracle/kernels.py).
Shapes follow the reference's tests (tests/models/test_gpt2.py:64-106, tests/kernels/test_transformer_fused.py:
182-205): GPT-2 caches [1024, 768], 12 heads, chunks not aligned to the 32-query block."""
import numpy as np
import pytest

from oracle import kernels as K

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(4321)
HEADS, CAP, D = 12, 1024, 768


def G(lk, a, dtype=np.float32):
    return lk.from_numpy(np.ascontiguousarray(a, dtype), device="gpu", copy=True)


def close(got, ref, tol):
    got = got.numpy() if hasattr(got, "numpy") else np.asarray(got)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got.astype(np.float64) - ref).max()
    scale = max(1.0, np.abs(ref).max())
    assert err <= tol * scale, f"max err {err:.3e} > {tol:.1e} * {scale:.3e}"


def _case(t):
    kc, vc = rng.standard_normal((CAP, D)), rng.standard_normal((CAP, D))
    qkv, bias = rng.standard_normal((t, 3 * D)), rng.standard_normal(3 * D) * 0.1
    return kc, vc, qkv, bias


@pytest.mark.parametrize("pos,t", [(0, 2), (0, 45), (6, 4), (5, 40), (100, 117), (37, 300), (1000, 24), (0, 512),
                                   (511, 33)])
def test_kv_write_rows_attention_cache(gpu, pos, t):
    lk = gpu
    kc, vc, qkv, bias = _case(t)
    KC, VC = G(lk, kc), G(lk, vc)
    P = G(lk, [pos], np.int64)
    Q, B = G(lk, qkv), G(lk, bias)
    rk, rv = K.kv_write_rows(kc.astype(np.float32), vc.astype(np.float32), qkv.astype(np.float32), pos,
                             bias.astype(np.float32))
    lk.ops.kv_write_rows_f32_gpu(KC, VC, Q, P, B)
    # written rows: one f32 add each; untouched rows bit-exact
    np.testing.assert_array_equal(KC.numpy(), rk.astype(np.float32))
    np.testing.assert_array_equal(VC.numpy(), rv.astype(np.float32))
    ref = K.attention_cache(qkv, rk, rv, pos, bias, HEADS)
    for _ in range(2):  # deterministic, no state
        got = lk.ops.attention_cache_f32_gpu(Q, KC, VC, P, B, HEADS)
        close(got, ref, 3e-5)
    close(lk.ops.attention_cache_sg_f32_gpu(Q, KC, VC, P, B, HEADS, nsg=8), ref, 3e-5)


@pytest.mark.parametrize("pos,t", [(0, 1), (300, 1), (1023, 1), (6, 4), (64, 64), (100, 117)])
def test_attention_gen(gpu, pos, t):
    """attention_gen / gen2 write the chunk's rows and attend over the cache: T = 1 through the split-key decode
    kernel, T > 1 through kv_write_rows + attention_cache."""
    lk = gpu
    kc, vc, qkv, bias = _case(t)
    rk, rv = K.kv_write_rows(kc, vc, qkv, pos, bias)
    ref = K.attention_cache(qkv, rk, rv, pos, bias, HEADS)
    for op in (lk.ops.attention_gen_f32_gpu, lk.ops.attention_gen2_f32_gpu):
        KC, VC = G(lk, kc), G(lk, vc)
        got = op(G(lk, qkv), KC, VC, G(lk, [pos], np.int64), G(lk, bias), HEADS)
        close(got, ref, 3e-5)
        close(KC, rk, 1e-6)
        close(VC, rv, 1e-6)


def test_rows_past_the_cache_are_dropped(gpu):
    """pos + T > cap: rows past the end are not written and their queries give NaN, the rows that fit are exact,
    and both kernels record LK_DEVERR_POSITION, raised at the next synchronisation (the reference's host kernel
    reports "pos + T exceeds the cache")."""
    from lokinfer_amd._lib import LokinferError, check_device_errors

    lk = gpu
    pos, t, fit = 1020, 8, 4
    kc, vc, qkv, bias = _case(t)
    KC, VC = G(lk, kc), G(lk, vc)
    P, Q, B = G(lk, [pos], np.int64), G(lk, qkv), G(lk, bias)
    lk.ops.kv_write_rows_f32_gpu(KC, VC, Q, P, B)
    with pytest.raises(LokinferError, match="device error 2: a position is outside the KV cache.*detail 1027"):
        check_device_errors()
    rk, rv = K.kv_write_rows(kc, vc, qkv[:fit], pos, bias)
    close(KC, rk, 1e-6)
    close(VC, rv, 1e-6)
    out = lk.ops.attention_cache_f32_gpu(Q, KC, VC, P, B, HEADS)
    with pytest.raises(LokinferError, match="device error 2"):
        check_device_errors()
    got = out.numpy()
    close(got[:fit], K.attention_cache(qkv[:fit], rk, rv, pos, bias, HEADS), 3e-5)
    assert np.isnan(got[fit:]).all()


@pytest.mark.parametrize("m", [1, 2, 10, 128, 512])
@pytest.mark.parametrize("k,splits", [(768, 2), (3072, 4)])
def test_gemm_auto_sk_ln2(gpu, m, k, splits):
    """The N = 768 projections of the chunk forward (reference tests/kernels/test_transformer_fused.py:182-205):
    split-K partials summed by add_bias_layernorm2_sk; both ops agree on how many planes hold data."""
    lk = gpu
    n = 768
    a, w = rng.standard_normal((m, k)), rng.standard_normal((k, n)) / np.sqrt(k)
    res = rng.standard_normal((m, n))
    bias, g, b = (rng.standard_normal(n) for _ in range(3))
    ref = K.gemm(a, w, bias) + res
    for op in (lk.ops.gemm_auto_sk_f32_gpu, lk.ops.gemm_splitk_f32_gpu):
        parts = op(G(lk, a), G(lk, w), splits)
        assert parts.shape == (splits, m, n)
        s, out = lk.ops.add_bias_layernorm2_sk_f32_gpu(parts, G(lk, bias), G(lk, res), G(lk, g), G(lk, b))
        close(s, ref, 2e-5)
        close(out, K.layernorm(ref, g, b, 1e-5), 1e-4)
        planes = lk.ops.splitk_planes(m, n, splits)
        pn = parts.numpy()
        if planes == 1:
            close(pn[0], K.gemm(a, w), 2e-5)
        else:  # each plane is its K range's product
            kc = k // splits
            for z in range(splits):
                close(pn[z], K.gemm(a[:, z * kc:(z + 1) * kc], w[z * kc:(z + 1) * kc]), 2e-5)


@pytest.mark.parametrize("m", [1, 7, 128])
def test_gemm_auto(gpu, m):
    lk = gpu
    k, n = 768, 3072
    x, w, b = rng.standard_normal((m, k)), rng.standard_normal((k, n)) / np.sqrt(k), rng.standard_normal(n)
    close(lk.ops.gemm_auto_f32_gpu(G(lk, x), G(lk, w)), K.gemm(x, w), 1e-5)
    close(lk.ops.gemm_auto_bias_gelu_f32_gpu(G(lk, x), G(lk, w), G(lk, b)), K.gemm(x, w, b, act="gelu"), 1e-5)


def test_arange_offset(gpu):
    lk = gpu
    out = lk.ops.arange_offset_i64_gpu(G(lk, [37], np.int64), 300).numpy()
    np.testing.assert_array_equal(out, 37 + np.arange(300))
