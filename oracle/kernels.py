"""TEST INFRASTRUCTURE ONLY. numpy float64 restatements of the GPU kernel ops of the reference's compiled path
(lariaus/lokinfer). Every function cites the reference kernel whose semantics it restates. Inputs may be any
float dtype; results are float64.
"""
from __future__ import annotations

import numpy as np

STAT_CHUNK = 128


def _d(x):
    return np.asarray(x, dtype=np.float64)


# ---- GEMM / GEMV (kernels/gpu/mps.mm:41-84; kokoro_lc.cpp:460-581; kokoro_tok.metal:878-924) ----------------

def gelu_tanh(v):
    """torch gelu(approximate='tanh') (kokoro_tok.metal:25-34)."""
    v = _d(v)
    return 0.5 * v * (1.0 + np.tanh(0.7978845608028654 * (v + 0.044715 * v ** 3)))


def gemm(a, b, bias=None, act="none", residual=None, scale=1.0, nt=False):
    """(act(a @ b + bias) + residual) * scale; nt: b given as b^T [N, K]."""
    a, b = _d(a), _d(b)
    y = a @ (b.T if nt else b)
    if bias is not None:
        y = y + _d(bias)
    if act == "relu":
        y = np.maximum(y, 0.0)
    elif act == "gelu":
        y = gelu_tanh(y)
    if residual is not None:
        y = y + _d(residual)
    return y * scale


# ---- transformer (kokoro_tok.metal:36-204, 465-876) -----------------------------------------------------------

def layernorm(x, gamma, beta, eps):
    """Biased-variance LayerNorm over the last dim (kokoro_tok.metal:169-204)."""
    x = _d(x)
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * _d(gamma) + _d(beta)


def add_bias_layernorm2(a, bias, r, gamma, beta, eps):
    """(s, LN(s)), s = a + bias + r (kokoro_tok.metal:79-117)."""
    s = _d(a) + _d(bias) + _d(r)
    return s, layernorm(s, gamma, beta, eps)


def attention_qkv(qkv, bias, heads, causal=False):
    """softmax((q + bq)(k + bk)^T / sqrt(64)) (v + bv) per head over fused qkv [T, 3D]
    (attention_qkv_sg_f32_gpu, kokoro_tok.metal:465-601; ops/kokoro_gpu.py:258-262)."""
    x = _d(qkv) + _d(bias)
    t, d3 = x.shape
    d = d3 // 3
    hd = d // heads
    out = np.zeros((t, d))
    for h in range(heads):
        q = x[:, h * hd:(h + 1) * hd]
        k = x[:, d + h * hd:d + (h + 1) * hd]
        v = x[:, 2 * d + h * hd:2 * d + (h + 1) * hd]
        s = q @ k.T / np.sqrt(hd)
        if causal:
            s = np.where(np.tril(np.ones((t, t), bool)), s, -np.inf)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        out[:, h * hd:(h + 1) * hd] = p @ v
    return out


def attention_decode(qkv, kc, vc, pos, bias, heads):
    """Writes k, v (+ bias) to row pos of copies of the caches, then one query over rows 0..pos
    (attention_decode_split_f32_gpu, transformer_gpu.cpp:122-222). Returns (out [1, D], kc', vc')."""
    x = _d(qkv)[0] + _d(bias)
    d = x.shape[0] // 3
    hd = d // heads
    kc, vc = _d(kc).copy(), _d(vc).copy()
    kc[pos] = x[d:2 * d]
    vc[pos] = x[2 * d:]
    out = np.zeros((1, d))
    for h in range(heads):
        q = x[h * hd:(h + 1) * hd]
        s = kc[:pos + 1, h * hd:(h + 1) * hd] @ q / np.sqrt(hd)
        p = np.exp(s - s.max())
        p /= p.sum()
        out[0, h * hd:(h + 1) * hd] = p @ vc[:pos + 1, h * hd:(h + 1) * hd]
    return out, kc, vc


def kv_write_rows(kc, vc, qkv, pos, bias):
    """Copies of the caches with rows pos..pos+T-1 = k, v of qkv [T, 3D] + bias (kv_write_rows_f32_gpu,
    python/lokinfer/ops/transformer.py:239-242; host form kernels/cpu/decode.cpp:115-128, which rejects
    pos + T > cap). Returns (kc', vc')."""
    x = _d(qkv) + _d(bias)
    t, d3 = x.shape
    d = d3 // 3
    kc, vc = _d(kc).copy(), _d(vc).copy()
    if pos < 0 or pos + t > kc.shape[0]:
        raise ValueError("kv_write_rows: pos + T exceeds the cache")
    kc[pos:pos + t] = x[:, d:2 * d]
    vc[pos:pos + t] = x[:, 2 * d:]
    return kc, vc


def attention_cache(qkv, kc, vc, pos, bias, heads):
    """Query i of qkv [T, 3D] (+ q bias) at position pos + i attends over cache rows 0..pos+i, scale 1/sqrt(64)
    (attention_cache_f32_gpu, python/lokinfer/ops/transformer.py:255-268; host form kernels/cpu/decode.cpp:130-175).
    The caches must already hold the chunk's rows."""
    x = _d(qkv) + _d(bias)
    kc, vc = _d(kc), _d(vc)
    t, d3 = x.shape
    d = d3 // 3
    hd = d // heads
    out = np.zeros((t, d))
    for h in range(heads):
        sl = slice(h * hd, (h + 1) * hd)
        for i in range(t):
            s = kc[:pos + i + 1, sl] @ x[i, sl] / np.sqrt(hd)
            p = np.exp(s - s.max())
            out[i, sl] = (p / p.sum()) @ vc[:pos + i + 1, sl]
    return out


# ---- Kokoro channel-last (kokoro_lc.metal:143-398) --------------------------------------------------------------

def channel_stats_lc(x):
    """Per-(128-row chunk, channel) (mean, M2) of x [L, C] -> [S, C, 2] (kokoro_lc.metal:172-208)."""
    x = _d(x)
    l, c = x.shape
    s = -(-l // STAT_CHUNK)
    out = np.zeros((s, c, 2))
    for i in range(s):
        blk = x[i * STAT_CHUNK:(i + 1) * STAT_CHUNK]
        m = blk.mean(0)
        out[i, :, 0] = m
        out[i, :, 1] = ((blk - m) ** 2).sum(0)
    return out


def adain_affine_lc(stats, gb, length, eps=1e-5):
    """[3, C] = (mean, (1 + g) / sqrt(var + eps), b) from chunk stats (exact chunk combine, biased var); channels
    >= len(gb) / 2 are (0, 0, 0) (kokoro_lc.metal:216-260)."""
    st = _d(stats)
    s, c, _ = st.shape
    n = np.array([min(STAT_CHUNK, length - i * STAT_CHUNK) for i in range(s)], np.float64)[:, None]
    mean = (st[:, :, 0] * n).sum(0) / length
    m2 = (st[:, :, 1] + n * (st[:, :, 0] - mean) ** 2).sum(0)
    var = m2 / length
    gb = _d(gb)
    cr = gb.shape[0] // 2
    af = np.zeros((3, c))
    af[0, :cr] = mean[:cr]
    af[1, :cr] = (1.0 + gb[:cr]) / np.sqrt(var[:cr] + eps)
    af[2, :cr] = gb[cr:]
    return af


def affine_act(x, affine=None, alpha=None, act="none", slope=0.0):
    """v = (x - af[0]) * af[1] + af[2] per channel, then snake v + sin^2(alpha v) / alpha or leaky
    (kokoro_lc.metal:151-166)."""
    v = _d(x)
    if affine is not None:
        af = _d(affine)
        v = (v - af[0]) * af[1] + af[2]
    if act == "snake":
        a = _d(alpha)
        v = v + np.sin(a * v) ** 2 / a
    elif act == "leaky":
        v = np.where(v >= 0, v, v * slope)
    return v


def conv1d_lc(x, w, b=None, padding=0, dilation=1, stride=1, residual=None, out_scale=1.0):
    """Channel-last conv1d: x [L, Ci], w [Co, K, Ci] -> [Lo, Co] = (conv + b [+ res]) * scale
    (conv1d_lc[_res]_f32_gpu, kokoro_lc.metal:62-128; ops/kokoro_gpu.py:20-54)."""
    x, w = _d(x), _d(w)
    l, ci = x.shape
    co, k, _ = w.shape
    xp = np.zeros((l + 2 * padding, ci))
    xp[padding:padding + l] = x
    lo = (l + 2 * padding - dilation * (k - 1) - 1) // stride + 1
    y = np.zeros((lo, co))
    for kk in range(k):
        rows = xp[kk * dilation: kk * dilation + (lo - 1) * stride + 1: stride]
        y += rows @ w[:, kk, :].T
    if b is not None:
        y += _d(b)
    if residual is not None:
        y += _d(residual)
    return y * out_scale


def convt_gather_lc(y, bias, kernel, stride, padding, add=None, reflect_left=False):
    """ConvTranspose1d overlap-add from y [Lin, K*Co] (y[j, kk*Co + co] = x[j] . W[:, co, kk]) + bias [+ add];
    reflect_left prepends F.pad(., (1, 0), 'reflect') (kokoro_lc.metal:262-286)."""
    y = _d(y)
    lin = y.shape[0]
    co = _d(bias).shape[0]
    full = (lin - 1) * stride + kernel
    acc = np.zeros((full, co))
    for j in range(lin):
        for kk in range(kernel):
            acc[j * stride + kk] += y[j, kk * co:(kk + 1) * co]
    out = acc[padding:full - padding] + _d(bias)
    if reflect_left:
        out = np.concatenate([out[1:2], out], 0)
    if add is not None:
        out = out + _d(add)
    return out


def dwconvt_lc(x, w, b, stride=2, padding=1):
    """Depthwise ConvTranspose1d, output_padding = stride - 1, channel-last (kokoro_lc.metal:333-348)."""
    x, w = _d(x), _d(w)
    lin, c = x.shape
    k = w.shape[1]
    full = (lin - 1) * stride + k + (stride - 1)
    acc = np.zeros((full + padding, c))
    for j in range(lin):
        for kk in range(k):
            acc[j * stride + kk] += x[j] * w[:, kk]
    lout = (lin - 1) * stride - 2 * padding + k + (stride - 1)
    return acc[padding:padding + lout] + _d(b)


def istft_logits(x_lc, n_fft=20, hop=5):
    """torch.istft(exp(mag) e^{i sin(phase)}, periodic Hann, center=True) from channel-last logits [L, Cpad]
    (istft_logits_lc_f32_gpu, kokoro_lc.metal:362-398; kokoro_signal.cpp:275-360)."""
    x = _d(x_lc)
    l = x.shape[0]
    bins = n_fft // 2 + 1
    spec = np.exp(x[:, :bins]) * np.exp(1j * np.sin(x[:, bins:2 * bins]))
    frames = np.fft.irfft(spec, n=n_fft, axis=1)  # [L, n_fft]
    win = 0.5 - 0.5 * np.cos(2 * np.pi * np.arange(n_fft) / n_fft)
    total = n_fft + hop * (l - 1)
    y = np.zeros(total)
    env = np.zeros(total)
    for t in range(l):
        y[t * hop:t * hop + n_fft] += frames[t] * win
        env[t * hop:t * hop + n_fft] += win ** 2
    pad = n_fft // 2
    return (y / np.where(env > 0, env, 1.0))[pad:pad + hop * (l - 1)]
