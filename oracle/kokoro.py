"""TEST INFRASTRUCTURE ONLY. PyTorch restatement of the Kokoro-82M forward with forced durations and explicit
SineGen noise: the semantics of the reference's graph (models/kokoro/model.py:619-785 in lariaus/lokinfer) and
of the Kokoro/StyleTTS2 modules it restates (ALBERT, DurationEncoder with AdaLayerNorm, shared BiLSTM,
AdainResBlk1d F0/N predictor, TextEncoder, Decoder with AdainResBlk1d blocks and the iSTFTNet Generator with
AdaINResBlock1 / Snake). The `kokoro` package is not available offline, so this is written from the module
definitions; it is also the CPU baseline of the bench (PyTorch f32 on the same model definition).

The harmonic source follows the reference kernel's op order (kernels/cpu/kokoro_signal.cpp:89-192): the
frame phase accumulated in double and rounded to f32, (phase * 2) * pi * 300 in f32, the x300 linear upsample as
fma(scale, i + 0.5, -0.5) and fma(t0, l0, t1 * l1), the 9-harmonic merge y += v * w[h] in order, then tanh.
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F

from lokinfer_amd.kokoro_weights import STYLE

SQRT1_2 = 1.0 / math.sqrt(2.0)


class Oracle:
    def __init__(self, sd: dict[str, np.ndarray], dtype=torch.float32):
        self.dt = dtype
        self.w = {k: torch.from_numpy(v).to(dtype) for k, v in sd.items()}
        self.sd = sd
        # set to [] to record every module call as (module name, type, input shape, output shape), the layout of
        # the reference's module-shape logs (bench/research/kokoro/shapes_*.json, written by forward hooks on
        # the Kokoro package's modules); None records nothing
        self.trace: list | None = None

    def _rec(self, name, kind, x, y):
        if self.trace is not None:
            self.trace.append((name, kind, list(x.shape), list(y.shape)))
        return y

    # ---- building blocks -----------------------------------------------------------------------------------
    def linear(self, x, p):
        return self._rec(p, "Linear", x, F.linear(x, self.w[p + ".weight"], self.w[p + ".bias"]))

    def lstm(self, x, p):
        """1-layer bidirectional nn.LSTM, x [T, I] -> [T, 2H] (reference lstm_bidir_f32_cpu, ops/kokoro.py:88-98)."""
        w = self.w
        hid = w[p + ".weight_hh_l0"].shape[1]
        m = torch.nn.LSTM(x.shape[1], hid, batch_first=True, bidirectional=True).to(self.dt)
        with torch.no_grad():
            for sfx in ("", "_reverse"):
                for n in ("weight_ih", "weight_hh", "bias_ih", "bias_hh"):
                    getattr(m, f"{n}_l0{sfx}").copy_(w[f"{p}.{n}_l0{sfx}"])
            return self._rec(p, "LSTM", x, m(x[None])[0][0])

    def adain(self, x, s, p):
        """AdaIN1d on channel-first x [C, L]: (1 + g) * instance_norm(x) + b, (g, b) = fc(s)."""
        h = self._rec(p + ".fc", "Linear", s, F.linear(s, self.w[p + ".fc.weight"], self.w[p + ".fc.bias"]))
        c = x.shape[0]
        g, b = h[:c], h[c:]
        return (1 + g[:, None]) * F.instance_norm(x[None], eps=1e-5)[0] + b[:, None]

    def conv(self, x, p, **kw):
        b = self.w.get(p + ".bias")
        return self._rec(p, "Conv1d", x, F.conv1d(x[None], self.w[p + ".weight"], b, **kw)[0])

    def resblk(self, x, s, p, upsample):
        """AdainResBlk1d (StyleTTS2), channel-first [C, L] (reference adain_resblk, model.py:141-157)."""
        r = F.leaky_relu(self.adain(x, s, p + ".norm1"), 0.2)
        if upsample:
            r = self._rec(p + ".pool", "ConvTranspose1d", r, F.conv_transpose1d(
                r[None], self.w[p + ".pool.weight"], self.w[p + ".pool.bias"], stride=2, padding=1, output_padding=1,
                groups=r.shape[0])[0])
        r = self.conv(r, p + ".conv1", padding=1)
        r = F.leaky_relu(self.adain(r, s, p + ".norm2"), 0.2)
        r = self.conv(r, p + ".conv2", padding=1)
        sc = F.interpolate(x[None], scale_factor=2, mode="nearest")[0] if upsample else x
        if p + ".conv1x1.weight" in self.w:
            sc = self.conv(sc, p + ".conv1x1")  # no bias
        return (r + sc) * SQRT1_2

    def resblock1(self, x, s, p, k):
        """AdaINResBlock1 with Snake, dilations 1, 3, 5 (reference adain_resblock1, model.py:208-219)."""
        for j, d in enumerate((1, 3, 5)):
            a1 = self.w[f"{p}.alpha1.{j}"].reshape(-1, 1)
            a2 = self.w[f"{p}.alpha2.{j}"].reshape(-1, 1)
            xt = self.adain(x, s, f"{p}.adain1.{j}")
            xt = xt + (1 / a1) * torch.sin(a1 * xt) ** 2
            xt = self.conv(xt, f"{p}.convs1.{j}", padding=d * (k - 1) // 2, dilation=d)
            xt = self.adain(xt, s, f"{p}.adain2.{j}")
            xt = xt + (1 / a2) * torch.sin(a2 * xt) ** 2
            xt = self.conv(xt, f"{p}.convs2.{j}", padding=(k - 1) // 2)
            x = xt + x
        return x

    # ---- stages --------------------------------------------------------------------------------------------
    def albert(self, ids):
        w, E = self.w, "bert.embeddings."
        t = ids.shape[0]
        e = w[E + "word_embeddings.weight"][ids] + w[E + "position_embeddings.weight"][:t]
        e = e + w[E + "token_type_embeddings.weight"][0]
        e = F.layer_norm(e, (128,), w[E + "LayerNorm.weight"], w[E + "LayerNorm.bias"], eps=1e-12)
        h = self.linear(e, "bert.encoder.embedding_hidden_mapping_in")
        L = "bert.encoder.albert_layer_groups.0.albert_layers.0."
        for _ in range(12):
            q, k, v = (self.linear(h, L + f"attention.{n}").view(t, 12, 64).transpose(0, 1) for n in
                       ("query", "key", "value"))
            a = F.scaled_dot_product_attention(q, k, v).transpose(0, 1).reshape(t, 768)
            a = self.linear(a, L + "attention.dense")
            h = F.layer_norm(h + a, (768,), w[L + "attention.LayerNorm.weight"], w[L + "attention.LayerNorm.bias"],
                             eps=1e-12)
            f = F.gelu(self.linear(h, L + "ffn"), approximate="tanh")
            f = self.linear(f, L + "ffn_output")
            h = F.layer_norm(f + h, (768,), w[L + "full_layer_layer_norm.weight"],
                             w[L + "full_layer_layer_norm.bias"], eps=1e-12)
        return h

    def duration_encoder(self, d_en, s_p):
        t = d_en.shape[0]
        sp = s_p[None].expand(t, STYLE)
        x = torch.cat([d_en, sp], 1)
        for i in range(3):
            x = self.lstm(x, f"predictor.text_encoder.lstms.{2 * i}")
            h = self.linear(s_p, f"predictor.text_encoder.lstms.{2 * i + 1}.fc")
            c = x.shape[1]
            x = (1 + h[:c]) * F.layer_norm(x, (c,), eps=1e-5) + h[c:]
            x = torch.cat([x, sp], 1)
        return x

    def f0n(self, en, s_p):
        sh = self.lstm(en, "predictor.shared").T  # [512, F]
        out = []
        for name in ("F0", "N"):
            y = self.resblk(sh, s_p, f"predictor.{name}.0", False)
            y = self.resblk(y, s_p, f"predictor.{name}.1", True)
            y = self.resblk(y, s_p, f"predictor.{name}.2", False)
            out.append(self.conv(y, f"predictor.{name}_proj")[0])
        return out

    def text_encoder(self, ids):
        w = self.w
        x = w["text_encoder.embedding.weight"][ids].T  # [512, T]
        for i in range(3):
            x = self.conv(x, f"text_encoder.cnn.{i}.0", padding=2)
            x = F.layer_norm(x.T, (x.shape[0],), w[f"text_encoder.cnn.{i}.1.gamma"], w[f"text_encoder.cnn.{i}.1.beta"],
                             eps=1e-5).T
            x = F.leaky_relu(x, 0.2)
        return self.lstm(x.T, "text_encoder.lstm")  # [T, 512]

    def decoder(self, asr, f0, n, s_d):
        f0d = self.conv(f0[None], "decoder.F0_conv", stride=2, padding=1)
        nd = self.conv(n[None], "decoder.N_conv", stride=2, padding=1)
        x = torch.cat([asr, f0d, nd], 0)
        x = self.resblk(x, s_d, "decoder.encode", False)
        asr_res = self.conv(asr, "decoder.asr_res.0")
        for i in range(4):
            x = torch.cat([x, asr_res, f0d, nd], 0)
            x = self.resblk(x, s_d, f"decoder.decode.{i}", i == 3)
        return x

    def harmonic_source(self, f0, noise):
        w = self.sd["decoder.generator.m_source.l_linear.weight"].reshape(9)
        b = self.sd["decoder.generator.m_source.l_linear.bias"]
        y = torch.from_numpy(harmonic_source(f0.detach().numpy().astype(np.float32), noise.numpy(), w, b)).to(self.dt)
        # the 9-harmonic merge inside is the source module's l_linear (9 -> 1), applied per sample
        self._rec("decoder.generator.m_source.l_linear", "Linear", noise, y[:, None])
        return y

    def stft(self, x):
        """TorchSTFT.transform as the reference computes it in f32 (stft_magphase, below) -> [22, frames]."""
        return torch.from_numpy(stft_magphase(x.detach().numpy().astype(np.float32))).to(self.dt)

    def stft_torch(self, x):
        """TorchSTFT.transform: magnitude and phase (angle) of torch.stft(n_fft 20, hop 5, periodic Hann,
        center, reflect) -> [22, frames]."""
        win = torch.hann_window(20, periodic=True, dtype=self.dt)
        z = torch.stft(x, 20, 5, 20, window=win, center=True, pad_mode="reflect", return_complex=True)
        # Frame 0 is even about its centre (reflect padding, periodic Hann), so its spectrum is exactly real; the
        # FFT's rounding-noise imaginary parts would make its phase +pi or -pi at random. Use the exact value.
        z[:, 0] = torch.complex(z[:, 0].real, torch.zeros_like(z[:, 0].real))
        return torch.cat([z.abs(), torch.angle(z)], 0)

    def generator(self, x, har, s_d, keep=None):
        G = "decoder.generator."
        rb = None
        for i, (k_up, u, k_noise) in enumerate(((20, 10, 7), (12, 6, 11))):
            x = F.leaky_relu(x, 0.1)
            xs = self.conv(har, G + f"noise_convs.{i}", **({"stride": 6, "padding": 3} if i == 0 else {}))
            if keep is not None:
                keep[f"xs{i}_conv"] = xs
            xs = self.resblock1(xs, s_d, f"{G}noise_res.{i}", k_noise)
            if keep is not None:
                keep[f"xs{i}"] = xs
            x = self._rec(G + f"ups.{i}", "ConvTranspose1d", x, F.conv_transpose1d(
                x[None], self.w[G + f"ups.{i}.weight"], self.w[G + f"ups.{i}.bias"], stride=u,
                padding=(k_up - u) // 2)[0])
            if i == 1:
                x = F.pad(x[None], (1, 0), mode="reflect")[0]
            x = x + xs
            if keep is not None:
                keep[f"ups{i}"] = x
            rb = [self.resblock1(x, s_d, f"{G}resblocks.{3 * i + j}", kk) for j, kk in enumerate((3, 7, 11))]
            x = (rb[0] + rb[1] + rb[2]) / 3
            if keep is not None:
                keep[f"stage{i}"] = x
        x = F.leaky_relu(x, 0.01)
        return self.conv(x, G + "conv_post", padding=3)  # [22, L1]

    def istft(self, post):
        spec = torch.exp(post[:11])
        phase = torch.sin(post[11:22])
        win = torch.hann_window(20, periodic=True, dtype=self.dt)
        return torch.istft(spec * torch.exp(phase * 1j), 20, 5, 20, window=win, center=True)

    @torch.no_grad()
    def forward(self, ids, ref_s, dur, noise, f0_override=None, stages=False):
        ids = torch.from_numpy(np.asarray(ids, np.int64))
        dur = torch.from_numpy(np.asarray(dur, np.int64))
        ref_s = torch.from_numpy(np.asarray(ref_s, np.float32)).to(self.dt)
        noise = torch.from_numpy(np.asarray(noise, np.float32))
        st = {}
        s_d, s_p = ref_s[:128], ref_s[128:]
        st["bert"] = bert = self.albert(ids)
        st["d_en"] = d_en = self.linear(bert, "bert_encoder")
        st["d"] = d = self.duration_encoder(d_en, s_p)
        st["en"] = en = torch.repeat_interleave(d, dur, 0)  # [F, 640]
        st["F0"], st["N"] = f0, n = self.f0n(en, s_p)
        st["t_en"] = t_en = self.text_encoder(ids)
        st["asr"] = asr = torch.repeat_interleave(t_en, dur, 0).T  # [512, F]
        st["dec"] = x = self.decoder(asr, f0, n, s_d)
        f0_src = f0 if f0_override is None else torch.as_tensor(f0_override).to(self.dt)
        st["har_source"] = har_source = self.harmonic_source(f0_src, noise)
        st["har"] = har = self.stft(har_source)
        st["post"] = post = self.generator(x, har, s_d, keep=st if stages else None)
        st["audio"] = self.istft(post)
        return st if stages else st["audio"]


def _fma32(a, b, c):
    """float32 fused multiply-add emulated in double (exact product, one rounding of the sum to double, then
    float32)."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)


def torch_remainder_1(a: np.ndarray) -> np.ndarray:
    """torch.remainder(a, 1.0) for float32: fmod, then + 1 when the sign differs (c10 BinaryOps)."""
    m = np.fmod(a, np.float32(1.0)).astype(np.float32)
    fix = (m != 0) & (m < 0)
    m[fix] = (m[fix] + np.float32(1.0)).astype(np.float32)
    return m


def harmonic_source(f0: np.ndarray, noise: np.ndarray, w: np.ndarray, b: np.ndarray) -> np.ndarray:
    """SourceModuleHnNSF(SineGen) with explicit noise f32[300 n, 9] -> f32[300 n] (reference
    harmonic_source_f32, kernels/cpu/kokoro_signal.cpp:89-192)."""
    f32 = np.float32
    n = f0.shape[0]
    f0 = f0.astype(f32)
    harm = np.arange(1, 10, dtype=f32)
    fn = (f0[:, None] * harm[None, :]).astype(f32)
    rad = torch_remainder_1((fn / f32(24000.0)).astype(f32))
    acc = np.cumsum(rad.astype(np.float64), axis=0)
    phase = ((acc.astype(f32) * f32(2.0)).astype(f32) * f32(math.pi)).astype(f32)
    p300 = (phase * f32(300.0)).astype(f32)  # [n, 9]
    s = n * 300
    i = np.arange(s, dtype=np.int64)
    scale = f32(1.0 / 300.0)
    real = _fma32(np.full(s, scale, f32), (i.astype(f32) + f32(0.5)).astype(f32), np.full(s, f32(-0.5)))
    real = np.maximum(real, f32(0.0))
    i0 = np.minimum(np.floor(real).astype(np.int64), n - 1)
    l1 = np.clip((real - i0.astype(f32)).astype(f32), f32(0.0), f32(1.0)).astype(f32)
    l0 = (f32(1.0) - l1).astype(f32)
    i1 = np.where(i0 < n - 1, i0 + 1, i0)
    t0, t1 = p300[i0], p300[i1]  # [s, 9]
    ph = _fma32(t0, np.repeat(l0[:, None], 9, 1), (t1 * l1[:, None]).astype(f32))
    sine = (np.sin(ph.astype(np.float64)).astype(f32) * f32(0.1)).astype(f32)
    fr = f0[i // 300]
    voiced = fr > f32(10.0)
    uv = voiced.astype(f32)[:, None]
    amp = np.where(voiced, f32(0.003), f32((f32(1.0) * f32(0.1)) / f32(3.0))).astype(f32)[:, None]
    v = ((sine * uv).astype(f32) + (amp * noise.astype(f32)).astype(f32)).astype(f32)
    y = np.zeros(s, f32)
    for h in range(9):
        y = (y + (v[:, h] * f32(w[h])).astype(f32)).astype(f32)
    return np.tanh((y + f32(b[0])).astype(np.float64)).astype(f32)


def stft_magphase(x: np.ndarray, n_fft: int = 20, hop: int = 5) -> np.ndarray:
    """(|X|, angle X) of the center = True, reflect-padded, periodic-Hann STFT of f32 x -> f32[2K, frames]
    (reference stft_magphase_f32, kernels/cpu/kokoro_signal.cpp:196-273): the windowed DFT table is built in
    double and rounded to f32, each bin accumulates re += tab[m] * frame[m] over m in order in f32, the DC and
    Nyquist bins (and every bin of the even-symmetric frame 0) are exactly real, |X| = sqrt(fma(re, re, im^2))."""
    f32 = np.float32
    x = x.astype(f32)
    s = x.shape[0]
    bins, pad = n_fft // 2 + 1, n_fft // 2
    frames = s // hop + 1
    m = np.arange(n_fft)
    win = (0.5 - 0.5 * np.cos(2.0 * np.pi * m / n_fft)).astype(f32)
    q = np.arange(frames)[:, None] * hop + m[None, :] - pad
    q = np.abs(q)
    q = np.where(q >= s, 2 * (s - 1) - q, q)
    fr = x[q]  # [frames, n_fft]
    out = np.zeros((2 * bins, frames), f32)
    for k in range(bins):
        ang = 2.0 * np.pi * ((k * m) % n_fft) / n_fft
        tre = (win.astype(np.float64) * np.cos(ang)).astype(f32)
        tim = (-win.astype(np.float64) * np.sin(ang)).astype(f32)
        re = np.zeros(frames, f32)
        im = np.zeros(frames, f32)
        for j in range(n_fft):
            re = (re + (tre[j] * fr[:, j]).astype(f32)).astype(f32)
            im = (im + (tim[j] * fr[:, j]).astype(f32)).astype(f32)
        if k == 0 or 2 * k == n_fft:
            im[:] = 0
        im[0] = 0
        out[k] = np.sqrt(_fma32(re, re, (im * im).astype(f32)))
        out[bins + k] = np.arctan2(im.astype(np.float64), re.astype(np.float64)).astype(f32)
    return out
