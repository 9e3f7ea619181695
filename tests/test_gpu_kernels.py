"""GPU parity of every kernel op against the CPU oracle (oracle/kernels.py), through the C-ABI registry
(ops.* -> lk_run_kernel). Tolerances follow the reference's kernel tests (tests/kernels/test_kokoro_gpu.py,
test_gemm_*.py, test_transformer_fused.py in lariaus/lokinfer): max |err| <= tol * max(1, max |ref|)."""
import numpy as np
import pytest
import torch

from oracle import kernels as K
from oracle import mnist

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(1234)


def G(lk, a):
    return lk.from_numpy(np.ascontiguousarray(a, np.float32), device="gpu", copy=True)


def close(got, ref, tol):
    got = got.numpy() if hasattr(got, "numpy") else np.asarray(got)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got.astype(np.float64) - ref).max() if ref.size else 0.0
    scale = max(1.0, np.abs(ref).max() if ref.size else 1.0)
    assert err <= tol * scale, f"max err {err:.3e} > {tol:.1e} * {scale:.3e}"


@pytest.mark.parametrize("m,n,k", [(1, 128, 784), (59, 2304, 768), (487, 768, 2048), (130, 70, 33), (256, 256, 512),
                                   (1000, 1536, 256), (487, 2304, 768), (487, 2048, 768), (100, 36, 20), (65, 68, 132),
                                   (2, 4, 4)])
def test_gemm(gpu, m, n, k):
    lk = gpu
    a, b = rng.standard_normal((m, k)), rng.standard_normal((k, n)) / np.sqrt(k)
    close(lk.ops.gemm_f32_gpu_mps(G(lk, a), G(lk, b)), K.gemm(a, b), 1e-5)


@pytest.mark.parametrize("m,n,k", [(1, 50257, 768), (3, 1000, 64), (200, 300, 96), (487, 2048, 640), (70, 45, 100),
                                   (1, 7, 4)])
def test_gemm_nt(gpu, m, n, k):
    lk = gpu
    a, b = rng.standard_normal((m, k)), rng.standard_normal((n, k)) / np.sqrt(k)
    close(lk.ops.gemm_nt_f32_gpu_mps(G(lk, a), G(lk, b)), K.gemm(a, b, nt=True), 1e-5)


@pytest.mark.parametrize("act", ["none", "relu", "gelu", "res"])
def test_gemm_epilogues(gpu, act):
    lk = gpu
    m, n, k = 77, 200, 160
    a, b, bias, r = rng.standard_normal((m, k)), rng.standard_normal((k, n)) / 12, rng.standard_normal(n), rng.standard_normal((m, n))
    A, B, BI, R = G(lk, a), G(lk, b), G(lk, bias), G(lk, r)
    if act == "res":
        got = lk.ops.gemm_steel_f32_gpu(A, B, BI, residual=R)
        ref = K.gemm(a, b, bias, residual=r)
    else:
        got = lk.ops.gemm_steel_f32_gpu(A, B, BI, act=act)
        ref = K.gemm(a, b, bias, act=act)
    close(got, ref, 1e-5)
    if act == "relu":
        close(lk.ops.gemm_bias_relu_f32_gpu(A, B, BI), ref, 1e-5)


@pytest.mark.parametrize("m,n,k", [(59, 768, 2048), (59, 2304, 768), (487, 768, 2048), (33, 100, 1000), (1, 64, 4096)])
@pytest.mark.parametrize("act", ["none", "relu", "gelu", "res"])
def test_gemm_split_k(gpu, m, n, k, act):
    """Few output tiles and a long K: K is split across workgroups (64-aligned ranges, partial tiles in the
    workspace) and a reduction applies the epilogue; same result as the one-pass kernel within f32 rounding."""
    lk = gpu
    a, b, bias, r = rng.standard_normal((m, k)), rng.standard_normal((k, n)) / np.sqrt(k), rng.standard_normal(n), rng.standard_normal((m, n))
    A, B, BI, R = G(lk, a), G(lk, b), G(lk, bias), G(lk, r)
    if act == "res":
        got = lk.ops.gemm_steel_f32_gpu(A, B, BI, residual=R)
        ref = K.gemm(a, b, bias, residual=r)
    else:
        got = lk.ops.gemm_steel_f32_gpu(A, B, BI, act=act)
        ref = K.gemm(a, b, bias, act=act)
    close(got, ref, 1e-5)
    close(lk.ops.gemm_f32_gpu_mps(A, B), K.gemm(a, b), 1e-5)


def test_mnist_mlp_plumbing(gpu):
    lk = gpu
    x, (w1, b1, w2, b2) = mnist.mlp_inputs(1)
    h = lk.ops.gemm_bias_relu_f32_gpu(G(lk, x), G(lk, w1), G(lk, b1))
    out = lk.ops.gemm_bias_f32_gpu(h, G(lk, w2), G(lk, b2))
    ref = mnist.mlp_forward(x, (w1, b1, w2, b2))
    got = out.numpy()
    assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()
    assert int(got.argmax()) == int(ref.argmax())


@pytest.mark.parametrize("n,k", [(2304, 768), (768, 768), (3072, 768), (768, 3072), (100, 40), (4, 1), (260, 130),
                                 (1028, 65)])
@pytest.mark.parametrize("variant", ["plain", "bias", "gelu", "res"])
def test_gemv4(gpu, n, k, variant):
    lk = gpu
    if n % 4:
        pytest.skip("gemv4 needs N % 4 == 0")
    x, w, b, r = rng.standard_normal((1, k)), rng.standard_normal((k, n)) / np.sqrt(k), rng.standard_normal(n), rng.standard_normal((1, n))
    X, W, B, R = G(lk, x), G(lk, w), G(lk, b), G(lk, r)
    for _ in range(3):  # repeated calls reuse the workspace
        if variant == "plain":
            got, ref = lk.ops.gemv4_f32_gpu(X, W), K.gemm(x, w)
        elif variant == "bias":
            got, ref = lk.ops.gemv4_f32_gpu(X, W, B), K.gemm(x, w, b)
        elif variant == "gelu":
            got, ref = lk.ops.gemv4_f32_gpu(X, W, B, act="gelu"), K.gemm(x, w, b, "gelu")
        else:
            got, ref = lk.ops.gemv4_f32_gpu(X, W, B, residual=R), K.gemm(x, w, b, residual=r)
        close(got, ref, 1e-5)


def test_gemv_rows_and_gemv1_bias(gpu):
    lk = gpu
    x, w = rng.standard_normal((1, 768)), rng.standard_normal((5000, 768)) / 28
    close(lk.ops.gemv_rows_f32_gpu(G(lk, x), G(lk, w)), K.gemm(x, w, nt=True), 1e-5)
    x2, w2, b2 = rng.standard_normal((333, 256)), rng.standard_normal((256, 1)), rng.standard_normal(1)
    close(lk.ops.gemv1_bias_f32_gpu(G(lk, x2), G(lk, w2), G(lk, b2)), K.gemm(x2, w2, b2), 1e-5)


@pytest.mark.parametrize("r,c", [(1, 768), (59, 768), (487, 768), (3, 2048), (5, 100)])
def test_layernorms(gpu, r, c):
    lk = gpu
    x, bias, res, g, b = (rng.standard_normal((r, c)), rng.standard_normal(c), rng.standard_normal((r, c)),
                          rng.standard_normal(c), rng.standard_normal(c))
    X, BI, RS, GG, BB = G(lk, x), G(lk, bias), G(lk, res), G(lk, g), G(lk, b)
    close(lk.ops.layernorm_f32_gpu(X, GG, BB, 1e-5), K.layernorm(x, g, b, 1e-5), 2e-5)
    close(lk.ops.add_bias_layernorm_f32_gpu(X, BI, RS, GG, BB), K.layernorm(x + bias + res, g, b, 1e-12), 2e-5)
    s, ln = lk.ops.add_bias_layernorm2_f32_gpu(X, BI, RS, GG, BB, 1e-5)
    rs, rl = K.add_bias_layernorm2(x, bias, res, g, b, 1e-5)
    close(s, rs, 1e-6)
    close(ln, rl, 2e-5)
    close(lk.ops.bias_gelu_f32_gpu(X, BI), K.gelu_tanh(x + bias), 1e-5)


@pytest.mark.parametrize("t", [1, 59, 130, 487])
@pytest.mark.parametrize("causal", [False, True])
def test_attention_qkv(gpu, t, causal):
    lk = gpu
    heads = 12
    qkv, bias = rng.standard_normal((t, 3 * 768)), rng.standard_normal(3 * 768) * 0.1
    got = lk.ops.attention_qkv_sg_f32_gpu(G(lk, qkv), G(lk, bias), heads, causal=causal)
    close(got, K.attention_qkv(qkv, bias, heads, causal), 1e-4)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_qkv_peaked(gpu, causal):
    """Scores spanning hundreds (near one-hot softmax rows, running max replaced many times across key tiles)."""
    lk = gpu
    t, heads = 333, 12
    qkv, bias = rng.standard_normal((t, 3 * 768)) * 4.0, rng.standard_normal(3 * 768)
    got = lk.ops.attention_qkv_f32_gpu(G(lk, qkv), G(lk, bias), heads, causal=causal)
    close(got, K.attention_qkv(qkv, bias, heads, causal), 1e-4)


@pytest.mark.parametrize("pos", [0, 1, 31, 32, 100, 512, 1023])
def test_attention_decode_split(gpu, pos):
    lk = gpu
    heads, cap, d = 12, 1024, 768
    kc, vc = rng.standard_normal((cap, d)), rng.standard_normal((cap, d))
    qkv, bias = rng.standard_normal((1, 3 * d)), rng.standard_normal(3 * d) * 0.1
    KC, VC = G(lk, kc), G(lk, vc)
    P = lk.from_numpy(np.array([pos], np.int64), device="gpu", copy=True)
    ref, rk, rv = K.attention_decode(qkv, kc, vc, pos, bias, heads)
    for _ in range(3):
        got = lk.ops.attention_decode_split_f32_gpu(G(lk, qkv), KC, VC, P, G(lk, bias), heads)
        close(got, ref, 3e-5)
    close(KC, rk, 1e-6)
    close(VC, rv, 1e-6)


# Caches past 128 chunks per head: each wave takes several 64-key chunks combined online (20000 rows: 3 chunks per
# wave, 105 waves per head); positions in the first, a middle (partly live) and the last wave.
@pytest.mark.parametrize("pos", [70, 8300, 19999])
def test_attention_decode_split_long_cache(gpu, pos):
    lk = gpu
    heads, cap, d = 4, 20000, 256
    kc, vc = rng.standard_normal((cap, d)), rng.standard_normal((cap, d))
    qkv, bias = rng.standard_normal((1, 3 * d)) * 2, rng.standard_normal(3 * d) * 0.1
    KC, VC = G(lk, kc), G(lk, vc)
    P = lk.from_numpy(np.array([pos], np.int64), device="gpu", copy=True)
    ref, rk, rv = K.attention_decode(qkv, kc, vc, pos, bias, heads)
    got = lk.ops.attention_decode_split_f32_gpu(G(lk, qkv), KC, VC, P, G(lk, bias), heads)
    close(got, ref, 3e-5)
    close(KC.numpy()[pos], rk[pos], 1e-6)
    close(VC.numpy()[pos], rv[pos], 1e-6)


@pytest.mark.parametrize("l,c", [(1, 64), (127, 256), (300, 1024), (2435, 128), (1000, 528)])
def test_stats_affine_act(gpu, l, c):
    lk = gpu
    x = rng.standard_normal((l, c)) * 2 + 0.5
    creal = c - 16 if c == 528 else c
    gb = rng.standard_normal(2 * creal) * 0.3
    alpha = np.abs(rng.standard_normal(c)) + 0.2
    X = G(lk, x)
    st = lk.ops.channel_stats_lc_f32_gpu(X)
    close(st, K.channel_stats_lc(x), 2e-5)
    af = lk.ops.adain_affine_lc_f32_gpu(st, G(lk, gb), l)
    ref_af = K.adain_affine_lc(K.channel_stats_lc(x), gb, l)
    if l > 1:
        close(af, ref_af, 2e-5)
    AF = G(lk, ref_af)
    close(lk.ops.snake_affine_lc_f32_gpu(X, AF, G(lk, alpha)), K.affine_act(x, ref_af, alpha, "snake"), 2e-5)
    close(lk.ops.leaky_lc_f32_gpu(X, 0.2, affine=AF), K.affine_act(x, ref_af, act="leaky", slope=0.2), 2e-5)
    close(lk.ops.leaky_lc_f32_gpu(X, 0.1), K.affine_act(x, act="leaky", slope=0.1), 1e-6)


def test_snake_wide_range(gpu):
    """Snake x + sin(a x)^2 / a over |a x| up to ~1e3: the kernel's pi-periodic reduction + hardware sine stays
    within 1e-6 of sin^2 evaluated in float64 at the same float32 product a x (plus the output's own rounding)."""
    lk = gpu
    l, c = 4096, 64
    x = np.concatenate([rng.uniform(-4, 4, (l // 2, c)), rng.uniform(-400, 400, (l // 2, c))]).astype(np.float32)
    alpha = rng.uniform(0.1, 3.0, c).astype(np.float32)
    af = np.stack([np.zeros(c), np.ones(c), np.zeros(c)]).astype(np.float32)  # identity affine
    got = lk.ops.snake_affine_lc_f32_gpu(G(lk, x), G(lk, af), G(lk, alpha)).numpy().astype(np.float64)
    y32 = (alpha[None, :] * x).astype(np.float32).astype(np.float64)
    inv = (np.float32(1) / alpha).astype(np.float64)
    ref = x.astype(np.float64) + inv[None, :] * np.sin(y32) ** 2
    err = np.abs(got - ref)
    tol = 1e-6 * np.maximum(1.0, inv[None, :]) + 2.0 ** -22 * np.abs(ref)
    assert (err <= tol).all(), f"max excess {np.max(err - tol):.3e}"


@pytest.mark.parametrize("l,ci,co,k,pad,dil", [(295, 528, 1024, 3, 1, 1), (600, 256, 256, 7, 9, 3), (1000, 128, 128, 11, 25, 5),
                                               (70, 1104, 512, 1, 0, 1), (33, 16, 64, 3, 1, 1), (5000, 128, 128, 3, 1, 1),
                                               (4888, 1104, 512, 1, 0, 1)])
def test_conv1d_lc(gpu, l, ci, co, k, pad, dil):
    lk = gpu
    x, w, b = rng.standard_normal((l, ci)), rng.standard_normal((co, k, ci)) / np.sqrt(k * ci), rng.standard_normal(co)
    ref = K.conv1d_lc(x, w, b, padding=pad, dilation=dil)
    close(lk.ops.conv1d_lc_f32_gpu(G(lk, x), G(lk, w), G(lk, b), padding=pad, dilation=dil), ref, 1e-4)
    r = rng.standard_normal(ref.shape)
    got = lk.ops.conv1d_lc_f32_gpu(G(lk, x), G(lk, w), G(lk, b), residual=G(lk, r), out_scale=0.5, padding=pad,
                                   dilation=dil)
    close(got, (ref + r) * 0.5, 1e-4)


@pytest.mark.parametrize("act", ["snake", "leaky", "none"])
def test_conv1d_act_lc(gpu, act):
    lk = gpu
    l, ci, co, k, d = 700, 128, 128, 7, 3
    x, w, b = rng.standard_normal((l, ci)), rng.standard_normal((co, k, ci)) / np.sqrt(k * ci), rng.standard_normal(co)
    af = np.stack([rng.standard_normal(ci) * 0.1, np.abs(rng.standard_normal(ci)) + 0.5, rng.standard_normal(ci) * 0.1])
    alpha = np.abs(rng.standard_normal(ci)) + 0.2
    h = K.affine_act(x, af, alpha, act, 0.2)
    res = rng.standard_normal((l, co))
    ref = K.conv1d_lc(h, w, b, padding=d * 3, dilation=d, residual=res)
    got = lk.ops.conv1d_act_lc_f32_gpu(G(lk, x), G(lk, w), G(lk, b), G(lk, af), G(lk, alpha), act=act, slope=0.2,
                                       residual=G(lk, res), padding=d * 3, dilation=d)
    close(got, ref, 1e-4)


def test_strided_conv(gpu):
    lk = gpu
    x, w, b = rng.standard_normal((1201, 32)), rng.standard_normal((256, 12, 32)) / 20, rng.standard_normal(256)
    ref = K.conv1d_lc(x, w, b, padding=3, stride=6)
    close(lk.ops.conv1d_lc_f32_gpu(G(lk, x), G(lk, w), G(lk, b), padding=3, stride=6), ref, 1e-4)


@pytest.mark.parametrize("lin,co,k,s,refl", [(59, 256, 20, 10, False), (590, 128, 12, 6, True), (3, 8, 4, 2, False)])
def test_convt_gather(gpu, lin, co, k, s, refl):
    lk = gpu
    y, b = rng.standard_normal((lin, k * co)), rng.standard_normal(co)
    p = (k - s) // 2
    ref = K.convt_gather_lc(y, b, k, s, p, reflect_left=refl)
    close(lk.ops.convt_gather_lc_f32_gpu(G(lk, y), G(lk, b), k, s, p, reflect_left=refl), ref, 1e-5)
    add = rng.standard_normal(ref.shape)
    close(lk.ops.convt_gather_lc_f32_gpu(G(lk, y), G(lk, b), k, s, p, add=G(lk, add), reflect_left=refl), ref + add, 1e-5)


def test_layout_glue(gpu):
    lk = gpu
    a, b = rng.standard_normal((50, 514)), rng.standard_normal((50, 66))
    got = lk.ops.concat_pad_lc_f32_gpu(G(lk, a), G(lk, b)).numpy()
    assert got.shape == (50, 592) and np.array_equal(got[:, :514], a.astype(np.float32))
    assert np.array_equal(got[:, 514:580], b.astype(np.float32)) and not got[:, 580:].any()
    assert lk.ops.concat_pad_lc_f32_gpu(G(lk, a)).shape == (50, 528)
    x = rng.standard_normal((77, 64)).astype(np.float32)
    assert np.array_equal(lk.ops.transpose_f32_gpu(G(lk, x)).numpy(), x.T)
    assert np.array_equal(lk.ops.lc_to_cf_f32_gpu(G(lk, x), 22).numpy(), x[:, :22].T)
    assert np.array_equal(lk.ops.upsample2_lc_f32_gpu(G(lk, x)).numpy(), np.repeat(x, 2, 0))
    y, z = rng.standard_normal((77, 64)).astype(np.float32), rng.standard_normal((77, 64)).astype(np.float32)
    close(lk.ops.add3_scale_f32_gpu(G(lk, x), G(lk, y), G(lk, z), 1 / 3), (x.astype(np.float64) + y + z) / 3, 1e-6)
    assert np.array_equal(lk.ops.add_f32_gpu(G(lk, x), G(lk, y)).numpy(), x + y)
    assert np.array_equal(lk.ops.mul_f32_gpu(G(lk, x), G(lk, y)).numpy(), x * y)
    w, bb = rng.standard_normal((64, 3)), rng.standard_normal(64)
    close(lk.ops.dwconvt_lc_f32_gpu(G(lk, x), G(lk, w), G(lk, bb)), K.dwconvt_lc(x, w, bb), 1e-5)


@pytest.mark.parametrize("l", [2, 3, 257, 3000])
def test_istft(gpu, l):
    lk = gpu
    x = rng.standard_normal((l, 64)) * 0.5
    close(lk.ops.istft_logits_lc_f32_gpu(G(lk, x)), K.istft_logits(x), 2e-5)


def test_graph_replay_matches_eager(gpu):
    lk = gpu
    a, b, bias = rng.standard_normal((300, 256)), rng.standard_normal((256, 512)) / 16, rng.standard_normal(512)
    w2 = rng.standard_normal((512, 768)) / 20

    def fn(x, w, bb, ww):
        h = lk.ops.gemm_bias_relu_f32_gpu(x, w, bb)
        return h, lk.ops.gemv4_f32_gpu(lk.ops.view(h, [1, 512], 0), ww)

    A, B, BI, W2 = G(lk, a), G(lk, b), G(lk, bias), G(lk, w2)
    e1, e2 = (t.numpy() for t in fn(A, B, BI, W2))
    m = lk.capture(fn)
    for _ in range(3):
        g1, g2 = (t.numpy() for t in m(A, B, BI, W2))
        torch.cuda.synchronize()
        assert np.array_equal(g1, e1) and np.array_equal(g2, e2)
        e1b = lk.ops.gemm_bias_relu_f32_gpu(A, B, BI).numpy()  # eager work between replays
        assert np.array_equal(e1b, e1)


def test_gemms_replay_in_graphs(gpu):
    """The plain / bias / relu / gelu / residual f32 GEMMs and the f16 bias / residual GEMMs, captured together in
    one graph at the models' shapes and at skinny large-K shapes (split K across workgroups, partials in the
    workspace), equal the eager results on every replay, with eager GEMMs between the replays."""
    lk = gpu
    F = lk.ops.f16_gpu
    f32 = [(59, 2048, 768, "none", True), (487, 768, 2304, "none", False), (487, 768, 2048, "gelu", False),
           (64, 8192, 256, "none", True), (16, 4096, 4096, "relu", False), (512, 768, 3072, "gelu", False)]
    ops32 = []
    for m, k, n, act, res in f32:
        ops32.append((G(lk, rng.standard_normal((m, k))), G(lk, rng.standard_normal((k, n)) / np.sqrt(k)),
                      G(lk, rng.standard_normal(n)), G(lk, rng.standard_normal((m, n))) if res else None, act))
    H = lambda a: lk.from_numpy(np.ascontiguousarray(a, dtype=np.float16), device="gpu", copy=True)
    x16 = [H(rng.standard_normal((mm, kk)) * 0.5) for mm, kk in ((416, 2048), (40, 6144))]
    w16 = [F.pack((rng.standard_normal((2048, 4096)) / 45).astype(np.float16)),
           F.pack((rng.standard_normal((6144, 2048)) / 78).astype(np.float16))]
    b16 = H(rng.standard_normal(4096))
    r16 = H(rng.standard_normal((40, 2048)))

    def fn():
        outs = [lk.ops.gemm_steel_f32_gpu(a, b, bias, act=act, residual=res) for a, b, bias, res, act in ops32]
        outs.append(F.gemm_bias_opt_f16_gpu(x16[0], w16[0], b16))
        outs.append(F.gemm_add_opt_f16_gpu(x16[1], w16[1], r16))
        return tuple(outs)

    eager = [t.numpy() for t in fn()]
    m = lk.capture(fn)
    for _ in range(4):  # the first call runs eagerly while the graph is captured, the others replay it
        got = [t.numpy() for t in m()]
        torch.cuda.synchronize()
        for i, (g, e) in enumerate(zip(got, eager)):
            assert np.array_equal(g.view(np.uint8), e.view(np.uint8)), i
        again = [t.numpy() for t in fn()]  # eager work between replays
        for i, (g, e) in enumerate(zip(again, eager)):
            assert np.array_equal(g.view(np.uint8), e.view(np.uint8)), i


@pytest.mark.parametrize("l,c,co,k,d,act", [(40001, 128, 128, 11, 5, "snake"), (33000, 128, 128, 3, 1, "snake"),
                                            (20000, 256, 256, 7, 3, "snake"), (30000, 128, 128, 7, 1, "leaky"),
                                            (32768, 512, 256, 3, 1, "none")])
def test_conv_tap_kernel_large(gpu, l, c, co, k, d, act):
    """Large-L convs take the taps-innermost halo kernel; check it against the oracle on a row sample."""
    lk = gpu
    x, w, b = rng.standard_normal((l, c)), rng.standard_normal((co, k, c)) / np.sqrt(k * c), rng.standard_normal(co)
    af = np.stack([rng.standard_normal(c) * 0.1, np.abs(rng.standard_normal(c)) + 0.5, rng.standard_normal(c) * 0.1])
    alpha = np.abs(rng.standard_normal(c)) + 0.2
    res = rng.standard_normal((l, co))
    pad = d * (k - 1) // 2
    got = lk.ops.conv1d_act_lc_f32_gpu(G(lk, x), G(lk, w), G(lk, b), G(lk, af), G(lk, alpha), act=act, slope=0.2,
                                       residual=G(lk, res), out_scale=0.5, padding=pad, dilation=d).numpy()
    rows = np.r_[0:300, l // 2 - 150:l // 2 + 150, l - 300:l]
    lo_in, hi_in = max(0, rows.min() - pad), rows.max() + pad + 1
    for seg in (slice(0, 300), slice(l // 2 - 150, l // 2 + 150), slice(l - 300, l)):
        s0, s1 = seg.start, seg.stop
        i0, i1 = max(0, s0 - pad), min(l, s1 + pad)
        h = K.affine_act(x[i0:i1], af, alpha, act, 0.2)
        full = K.conv1d_lc(np.pad(h, ((pad - (s0 - i0), pad - (i1 - s1)), (0, 0))), w, b, padding=0, dilation=d)
        ref = (full + res[s0:s1]) * 0.5
        close(got[s0:s1], ref, 1e-4)
    del lo_in, hi_in


@pytest.mark.parametrize("k,n", [(768, 2304), (3072, 768), (100, 36)])
def test_gemv_partial_reduce_ln(gpu, k, n):
    lk = gpu
    x, w = rng.standard_normal((1, k)), rng.standard_normal((k, n)) / np.sqrt(k)
    bias, res, g, b = rng.standard_normal(n), rng.standard_normal((1, n)), rng.standard_normal(n), rng.standard_normal(n)
    part = lk.ops.gemv_partial_f32_gpu(G(lk, x), G(lk, w))
    assert part.shape == (lk.ops.gemv_partial_slices(k), n)
    close(part.numpy().sum(0)[None], K.gemm(x, w), 1e-5)
    if n <= 1024:
        s, ln = lk.ops.reduce_bias_res_ln2_f32_gpu(part, G(lk, bias), G(lk, res), G(lk, g), G(lk, b), 1e-5)
        rs, rl = K.add_bias_layernorm2(K.gemm(x, w), bias, res, g, b, 1e-5)
        close(s, rs, 1e-5)
        close(ln, rl, 2e-5)


def test_gemv_partial_gelu(gpu):
    lk = gpu
    k0, k, n = 768, 3072, 768
    x, w1, b1 = rng.standard_normal((1, k0)), rng.standard_normal((k0, k)) / np.sqrt(k0), rng.standard_normal(k) * 0.1
    w2 = rng.standard_normal((k, n)) / np.sqrt(k)
    p1 = lk.ops.gemv_partial_f32_gpu(G(lk, x), G(lk, w1))
    p2 = lk.ops.gemv_partial_gelu_f32_gpu(p1, G(lk, b1), G(lk, w2))
    ref = K.gemm(K.gelu_tanh(K.gemm(x, w1, b1)), w2)
    close(p2.numpy().sum(0)[None], ref, 1e-5)


@pytest.mark.parametrize("pos", [0, 63, 64, 511, 1023])
def test_attention_decode_part(gpu, pos):
    lk = gpu
    heads, d, cap = 12, 768, 1024
    x = rng.standard_normal((1, d))
    w = rng.standard_normal((d, 3 * d)) / np.sqrt(d)
    bias = rng.standard_normal(3 * d) * 0.1
    kc, vc = rng.standard_normal((cap, d)), rng.standard_normal((cap, d))
    wo = rng.standard_normal((d, d)) / np.sqrt(d)
    KC, VC = G(lk, kc), G(lk, vc)
    qp = lk.ops.gemv_partial_f32_gpu(G(lk, x), G(lk, w))
    ch = lk.ops.attention_decode_part_f32_gpu(qp, KC, VC, lk.from_numpy(np.array([pos], np.int64), device="gpu", copy=True),
                                            G(lk, bias), heads)
    op = lk.ops.gemv_partial_attn_f32_gpu(ch, G(lk, wo))
    att, kref, vref = K.attention_decode(K.gemm(x, w), kc, vc, pos, bias, heads)
    close(op.numpy().sum(0)[None], K.gemm(att, wo), 1e-5)
    close(KC.numpy()[pos], kref[pos], 1e-6)
    close(VC.numpy()[pos], vref[pos], 1e-6)


def test_gemv_partial_res_ln(gpu):
    lk = gpu
    k, n = 768, 2304
    x, w0 = rng.standard_normal((1, 3072)), rng.standard_normal((3072, k)) / 55
    bias, res, g, b = rng.standard_normal(k), rng.standard_normal((1, k)), rng.standard_normal(k), rng.standard_normal(k)
    w = rng.standard_normal((k, n)) / np.sqrt(k)
    xp = lk.ops.gemv_partial_f32_gpu(G(lk, x), G(lk, w0))
    part, s = lk.ops.gemv_partial_res_ln_f32_gpu(xp, G(lk, bias), G(lk, res), G(lk, g), G(lk, b), G(lk, w), 1e-5)
    rs, rl = K.add_bias_layernorm2(K.gemm(x, w0), bias, res, g, b, 1e-5)
    close(s, rs, 1e-5)
    close(part.numpy().sum(0)[None], K.gemm(rl, w), 2e-5)
    part2, x2 = lk.ops.gemv_partial_ln_f32_gpu(G(lk, res), G(lk, g), G(lk, b), G(lk, w), 1e-5)
    close(x2, res.astype(np.float32), 0)
    close(part2.numpy().sum(0)[None], K.gemm(K.layernorm(res, g, b, 1e-5), w), 2e-5)


def test_gemv_partial_embed_ln(gpu):
    lk = gpu
    v, p, k, n = 97, 40, 768, 2304
    wte, wpe = rng.standard_normal((v, k)), rng.standard_normal((p, k))
    g, b = rng.standard_normal(k), rng.standard_normal(k)
    w = rng.standard_normal((k, n)) / np.sqrt(k)
    WTE, WPE = G(lk, wte), G(lk, wpe)
    ids = lambda i: lk.from_numpy(np.array([i], np.int64), device="gpu", copy=True)
    for tok, pos in ((5, 0), (96, 39)):
        part, s = lk.ops.gemv_partial_embed_ln_f32_gpu(WTE, ids(tok), WPE, ids(pos), G(lk, g), G(lk, b), G(lk, w),
                                                       1e-5)
        h = (wte[tok].astype(np.float32) + wpe[pos].astype(np.float32))[None]
        close(s, h, 0)  # one f32 add per element: exact
        close(part.numpy().sum(0)[None], K.gemm(K.layernorm(h, g, b, 1e-5), w), 2e-5)
    part, s = lk.ops.gemv_partial_embed_ln_f32_gpu(WTE, ids(v), WPE, ids(0), G(lk, g), G(lk, b), G(lk, w), 1e-5)
    with pytest.raises(lk.LokinferError, match="device error 3"):
        s.numpy()


@pytest.mark.parametrize("v", [50257, 10, 4099])
def test_lm_head_ln_argmax(gpu, v):
    lk = gpu
    k = 768
    x, w0 = rng.standard_normal((1, 3072)), rng.standard_normal((3072, k)) / 55
    bias, res, g, b = rng.standard_normal(k), rng.standard_normal((1, k)), rng.standard_normal(k), rng.standard_normal(k)
    table = rng.standard_normal((v, k)) * 0.02
    xp = lk.ops.gemv_partial_f32_gpu(G(lk, x), G(lk, w0))
    logits, am = lk.ops.lm_head_ln_argmax_f32_gpu(xp, G(lk, bias), G(lk, res), G(lk, g), G(lk, b), G(lk, table), 1e-5)
    _, ln = K.add_bias_layernorm2(K.gemm(x, w0), bias, res, g, b, 1e-5)
    ref = K.gemm(ln, table, nt=True)
    close(logits, ref, 2e-5)
    got = logits.numpy()
    assert am.numpy().tolist() == [int(np.argmax(got[0]))]
    assert int(am.numpy()[0]) == int(np.argmax(ref[0]))
    if v > 3000:
        # ties go to the first index: copy the winning row to a lower and a higher index
        t2 = table.copy()
        best = int(np.argmax(ref[0]))
        t2[3] = t2[best]
        t2[v - 1] = t2[best]
        logits2, am2 = lk.ops.lm_head_ln_argmax_f32_gpu(xp, G(lk, bias), G(lk, res), G(lk, g), G(lk, b), G(lk, t2),
                                                        1e-5)
        l2 = logits2.numpy()[0]
        assert l2[3] == l2[best] == l2[v - 1]
        assert am2.numpy().tolist() == [3]


# At least 256 output tiles of 128 x 128: the only shapes that select convTapKernel<128, 128>, whose epilogue
# writes the 128-row channel statistics itself (the Kokoro-487 decoder and generator sizes).
@pytest.mark.parametrize("l,ci,co,k,dil,act", [(5000, 1104, 1024, 3, 1, "leaky"), (40000, 128, 128, 7, 3, "snake"),
                                               (33000, 128, 128, 11, 5, "none")])
def test_conv1d_tap128_stats(gpu, l, ci, co, k, dil, act):
    lk = gpu
    assert -(-l // 128) * -(-co // 128) >= 256
    x, w, b = rng.standard_normal((l, ci)), rng.standard_normal((co, k, ci)) / np.sqrt(k * ci), rng.standard_normal(co)
    af = np.stack([rng.standard_normal(ci) * 0.1, np.abs(rng.standard_normal(ci)) + 0.5, rng.standard_normal(ci) * 0.1])
    alpha = np.abs(rng.standard_normal(ci)) + 0.2
    pad = dil * (k - 1) // 2
    res = rng.standard_normal((l, co))
    ref = K.conv1d_lc(K.affine_act(x, af, alpha, act, 0.2), w, b, padding=pad, dilation=dil, residual=res,
                      out_scale=0.7071)
    y, st = lk.ops.conv1d_act_lc_f32_gpu(G(lk, x), G(lk, w), G(lk, b), G(lk, af), G(lk, alpha), act=act, slope=0.2,
                                         residual=G(lk, res), out_scale=0.7071, padding=pad, dilation=dil, stats=True)
    close(y, ref, 1e-4)
    np.testing.assert_allclose(st.numpy(), K.channel_stats_lc(y.numpy()), rtol=1e-4, atol=1e-4)
