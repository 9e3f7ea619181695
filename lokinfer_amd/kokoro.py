"""Kokoro-82M forward on the MI355X kernels, GPU-resident end to end: the graph of the reference's
`build(sd, gpu=True, forced_durations=True, explicit_noise=True)` (models/kokoro/model.py:619-785 in
lariaus/lokinfer) with every stage on the device.

Inputs: ids i64[T] (pad id 0 at both ends), ref_s f32[256], dur i64[T] (forced durations), noise f32[600 F, 9]
(the SineGen noise; F = sum(dur) frames). Output: audio f32[600 F].

Stages (channel-last [L, C] at frame rate, [T, C] at token rate):
  ALBERT x12 (shared weights): MFMA GEMMs + flash attention + fused add/bias/LayerNorm   (model.py:583-610)
  bert_encoder, DurationEncoder (3 BiLSTM + AdaLayerNorm), repeat_interleave by dur     (model.py:649-680)
  shared BiLSTM -> F0 / N curves (3 AdainResBlk1d each + one-column projection)          (model.py:387-401)
  TextEncoder (3 x conv k5 + LN + leaky, BiLSTM) -> asr                                   (model.py:591-603)
  Decoder: F0_conv / N_conv, encode + 4 decode AdainResBlk1d                             (model.py:369-380)
  Generator: harmonic source + STFT, noise convs, 2 x (noise_res, convT, 3 resblocks), conv_post, iSTFT
                                                                                          (model.py:479-508)
Where the reference keeps work on the host CPU (LSTMs, embeddings, alignment, harmonic source, STFT, strided and
single-channel convs, the ALBERT embeddings) this backend runs device kernels, so a forward is one captured HIP
graph with no host round trips. The generator's Snake resblock convs run as the Winograd pair (input transform
with AdaIN affine + Snake fused, per-point MFMA GEMM with the channel statistics in its epilogue) when the grid
is large enough, as the reference does; every other conv is one implicit-GEMM MFMA kernel with the affine and
activation fused into its operand staging.

The durations predictor (predictor.lstm + duration_proj) is not computed: with forced durations its output is
unused, and the reference's dead-code pass removes it from the compiled graph as well.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import ops, winograd
from .compiler import capture as lk_capture
from .runtime import GpuContext
from .tensor import Tensor, from_numpy

SQRT1_2 = 1.0 / math.sqrt(2.0)


def _pad16(n: int) -> int:
    return -(-n // 16) * 16


def _w_lc(a: np.ndarray, ci_pad: int | None = None) -> np.ndarray:
    """torch conv weight [Co, Ci, K] -> channel-last [Co, K, Ci_pad] (zero input channels past Ci)."""
    co, ci, k = a.shape
    cp = ci_pad or _pad16(ci)
    out = np.zeros((co, k, cp), np.float32)
    out[:, :, :ci] = a.transpose(0, 2, 1)
    return out


def _w_convt(a: np.ndarray) -> np.ndarray:
    """ConvTranspose1d weight [Ci, Co, K] -> [Ci, K * Co] (GEMM, then the overlap-add gather)."""
    ci, co, k = a.shape
    return np.ascontiguousarray(a.transpose(0, 2, 1).reshape(ci, k * co))


def _w_convt_nt(a: np.ndarray) -> np.ndarray:
    """ConvTranspose1d weight [Ci, Co, K] -> [K * Co, Ci], the NT GEMM's form of _w_convt (its transpose)."""
    return np.ascontiguousarray(_w_convt(a).T)


def _vec_pad(a: np.ndarray, n: int) -> np.ndarray:
    out = np.zeros(n, np.float32)
    out[: a.shape[0]] = a
    return out


class KokoroGpu:
    """The Kokoro forward on the GPU. runtime="capture" replays a torch stream capture of the function with its
    concurrent side-stream branches; runtime="compiled" traces it into the runtime's IR (lk.compile) per (T, F)
    signature and runs it from the C++ executable (save() writes that model as a .lkm), its graph's independent
    branches on up to `lanes` concurrent lanes. The conv dispatch (Winograd or tap conv) depends on the lengths,
    so the traced model is specialized per signature."""

    def __init__(self, sd: dict[str, np.ndarray], graph: bool = True, runtime: str = "capture", lanes: int = 6):
        if runtime not in ("capture", "compiled"):
            raise ValueError("runtime must be 'capture' or 'compiled'")
        self.runtime = runtime
        self.lanes = lanes
        self._compiled: dict[tuple, object] = {}
        self.sd = sd
        self._g: dict[str, Tensor] = {}
        self._per_t: dict[tuple, Tensor] = {}
        self.banks = {root: self._bank(root) for root in ("predictor", "decoder")}
        # side streams for the graph's concurrent branches (default priority)
        self.streams = [torch.cuda.Stream() for _ in range(4)]
        self.model = lk_capture(self._forward, graph=graph)
        self.debug: dict | None = None  # set to {} to keep named intermediates (eager runs only)

    def _keep(self, name: str, t: Tensor) -> None:
        if self.debug is not None:
            self.debug[name] = t

    # ---- weights (uploaded once) ------------------------------------------------------------------------
    def g(self, key: str, fn=None) -> Tensor:
        k = key if fn is None else f"{key}#{fn.__name__}"
        t = self._g.get(k)
        if t is None:
            a = self.sd[key] if fn is None else fn(self.sd[key])
            t = from_numpy(np.ascontiguousarray(a, dtype=np.float32), device="gpu", copy=True)
            self._g[k] = t
        return t

    def const(self, key: str, make) -> Tensor:
        t = self._g.get(key)
        if t is None:
            t = from_numpy(np.ascontiguousarray(make(), dtype=np.float32), device="gpu", copy=True)
            self._g[key] = t
        return t

    def _bank(self, root: str):
        """All `<root>.*.fc` style projections as one [128, total] weight (one GEMV per style vector), with each
        fc's (offset, width) (reference W.style_bank, model.py:67-81)."""
        names = sorted(k[: -len(".weight")] for k in self.sd if k.startswith(root + ".") and k.endswith(".fc.weight"))
        wt = np.concatenate([self.sd[n + ".weight"].T for n in names], axis=1)
        b = np.concatenate([self.sd[n + ".bias"] for n in names])
        offs, o = {}, 0
        for n in names:
            offs[n] = (o, self.sd[n + ".bias"].shape[0])
            o += offs[n][1]
        return (from_numpy(np.ascontiguousarray(wt), device="gpu", copy=True),
                from_numpy(np.ascontiguousarray(b), device="gpu", copy=True), offs)

    def lstm_w(self, p: str):
        key = p + "#lstm"
        if key not in self._g:
            sd = self.sd
            w_ih = np.concatenate([sd[p + ".weight_ih_l0"], sd[p + ".weight_ih_l0_reverse"]])
            w_hh_t = np.concatenate([sd[p + ".weight_hh_l0"], sd[p + ".weight_hh_l0_reverse"]]).T
            b = np.concatenate([sd[p + ".bias_ih_l0"] + sd[p + ".bias_hh_l0"],
                                sd[p + ".bias_ih_l0_reverse"] + sd[p + ".bias_hh_l0_reverse"]])
            self._g[key] = tuple(from_numpy(np.ascontiguousarray(a, np.float32), device="gpu", copy=True)
                                 for a in (w_ih, w_hh_t, b))
        return self._g[key]

    def per_t(self, kind: str, n: int, make) -> Tensor:
        """Shape-dependent constants (positions 0..T-1, zero rows), built on the eager warm-up call so that the
        captured graph only reads them."""
        key = (kind, n)
        t = self._per_t.get(key)
        if t is None:
            t = make()
            self._per_t[key] = t
        return t

    # ---- building blocks ------------------------------------------------------------------------------------
    def style(self, bank, prefix: str) -> Tensor:
        vec, offs = bank
        off, n = offs[prefix]
        return ops.view(vec, [n], off)

    def affine(self, x: Tensor, bank, prefix: str, stats: Tensor | None = None, dilation: int = 1) -> Tensor:
        st = ops.channel_stats_lc_f32_gpu(x) if stats is None else stats
        if dilation > 1:  # statistics of a dilated Winograd conv: chunks per residue class
            return ops.wino_adain_affine_lc_f32_gpu(st, self.style(bank, prefix), x.shape[0], dilation=dilation)
        return ops.adain_affine_lc_f32_gpu(st, self.style(bank, prefix), length=x.shape[0])

    def resblk(self, x: Tensor, bank, p: str, cin: int, cout: int, upsample: bool) -> Tensor:
        """AdainResBlk1d, channel-last x f32[L, pad16(cin)] (padding channels stay 0)."""
        af = self.affine(x, bank, p + ".norm1.fc")
        cp = _pad16(cin)
        if upsample:
            h = ops.leaky_lc_f32_gpu(x, 0.2, affine=af)
            h = ops.dwconvt_lc_f32_gpu(h, self.const(p + "#pool_w", lambda: _pool_pad(self.sd[p + ".pool.weight"], cp)),
                                       self.const(p + "#pool_b", lambda: _vec_pad(self.sd[p + ".pool.bias"], cp)))
            h, hst, hd = self.conv(h, p + ".conv1", None, 3, stats=True)
        else:
            h, hst, hd = self.conv(x, p + ".conv1", af, 3, act="leaky", slope=0.2, stats=True)
        af2 = self.affine(h, bank, p + ".norm2.fc", hst, hd)
        sc = ops.upsample2_lc_f32_gpu(x) if upsample else x
        if p + ".conv1x1.weight" in self.sd:
            sc = ops.conv1d_lc_f32_gpu(sc, self.g(p + ".conv1x1.weight", _w_lc),
                                       self.const(f"zeros#{cout}", lambda: np.zeros(cout)))
        return self.conv(h, p + ".conv2", af2, 3, act="leaky", slope=0.2, residual=sc, out_scale=SQRT1_2)[0]

    def wino(self, key: str, ci_pad: int, co_pad: int):
        """(Ut, tr) of conv weight `key` for the Winograd ops (U transposed, the ops' u_layout 1), input channels
        zero-padded to ci_pad and output channels to co_pad, transformed once on the host."""
        k = f"{key}#wino{ci_pad}x{co_pad}"
        if k not in self._g:
            w = self.sd[key]
            wp = np.zeros((co_pad, ci_pad, w.shape[2]), np.float32)
            wp[: w.shape[0], : w.shape[1]] = w
            u, tr = winograd.wino_weights_t(wp)
            self._g[k] = (from_numpy(u, device="gpu", copy=True), from_numpy(tr, device="gpu", copy=True))
        return self._g[k]

    def conv(self, x: Tensor, p: str, af: Tensor | None, k: int, d: int = 1, act: str = "none", alpha=None,
             slope: float = 0.0, residual=None, out_scale: float = 1.0, stats: bool = False, co_pad: int = 0):
        """conv(act(affine(x))) (+ residual) * out_scale, optionally with the output's channel statistics, on the
        Winograd pair or the tap conv, whichever is faster at this shape. Measured on MI355X over every conv of the
        59- and 487-token forwards: the pair (transform + GEMM) costs at least ~55-60 us, the K = 3 tap conv ~55-60
        us per 1e9 multiply-adds, and K >= 7 favours Winograd once its grid of 64-tile x 64-channel workgroups
        reaches 64. co_pad > Co: output channels past Co are zero (zero weights and bias). Returns (y, stats,
        stats_dilation): Winograd statistics come per residue class of the dilation."""
        co, ci = self.sd[p + ".weight"].shape[:2]
        cop = max(co, co_pad)
        grid = (cop // 64) * -(-(-(-x.shape[0] // d)) // 256) * d
        pad = d * (k - 1) // 2
        bias = self.g(p + ".bias") if cop == co else self.const(f"{p}.bias#pad{cop}",
                                                                 lambda: _vec_pad(self.sd[p + ".bias"], cop))
        macs = x.shape[0] * ci * cop * k
        if cop % 64 == 0 and (macs >= 1_000_000_000 or (k >= 7 and grid >= 64)):
            u, tr = self.wino(p + ".weight", x.shape[1], cop)
            kw = {"alpha": alpha} if act == "snake" else {"slope": slope} if act == "leaky" else {}
            y = ops.conv1d_wino_lc_f32_gpu(x, u, bias, tr, k, residual=residual, out_scale=out_scale,
                                           padding=pad, dilation=d, affine=af if act != "none" else None,
                                           stats=stats, u_layout=1, **kw)
            return (y + (d,)) if stats else (y, None, 1)
        w = self.g(p + ".weight", _w_lc) if cop == co else self.const(
            f"{p}#lc{cop}", lambda: _w_lc(np.concatenate([self.sd[p + ".weight"],
                                                          np.zeros((cop - co, *self.sd[p + ".weight"].shape[1:]),
                                                                   np.float32)])))
        if af is None:
            cp = x.shape[1]
            af = self.const(f"identity_affine{cp}", lambda: np.stack([np.zeros(cp), np.ones(cp), np.zeros(cp)]))
        y = ops.conv1d_act_lc_f32_gpu(x, w, bias, af, alpha, act=act, slope=slope, padding=pad, dilation=d, residual=residual, out_scale=out_scale,
                                      stats=stats)
        return (y + (1,)) if stats else (y, None, 1)

    def resblock1(self, x: Tensor, bank, p: str, k: int, x_stats: Tensor | None = None) -> Tensor:
        """AdaINResBlock1 (Snake), dilations 1, 3, 5; every conv has AdaIN affine + Snake fused in its prologue."""
        st, sd = (ops.channel_stats_lc_f32_gpu(x) if x_stats is None else x_stats), 1
        for j, d in enumerate((1, 3, 5)):
            af = self.affine(x, bank, f"{p}.adain1.{j}.fc", st, sd)
            h, hst, hd = self.conv(x, f"{p}.convs1.{j}", af, k, d, "snake", alpha=self.g(f"{p}.alpha1.{j}", _flat),
                                   stats=True)
            af2 = self.affine(h, bank, f"{p}.adain2.{j}.fc", hst, hd)
            x, st, sd = self.conv(h, f"{p}.convs2.{j}", af2, k, 1, "snake", alpha=self.g(f"{p}.alpha2.{j}", _flat),
                                  residual=x, stats=j < 2)
        return x

    def noise_block(self, har: Tensor, bank, i: int) -> Tensor:
        """noise_convs.i (stride 6 for stage 0, 1x1 for stage 1) then noise_res.i (AdaINResBlock1, K = 7 / 11)."""
        G = "decoder.generator."
        xs = ops.conv1d_lc_f32_gpu(har, self.g(G + f"noise_convs.{i}.weight", _w_lc_32),
                                   self.g(G + f"noise_convs.{i}.bias"), **({"stride": 6, "padding": 3} if i == 0 else {}))
        self._keep(f"xs{i}_conv", xs)
        xs = self.resblock1(xs, bank, f"{G}noise_res.{i}", (7, 11)[i])
        self._keep(f"xs{i}", xs)
        return xs

    def lstm(self, x: Tensor, p: str) -> Tensor:
        return ops.lstm_bidir_t_f32_gpu(x, *self.lstm_w(p))

    # ---- stages ---------------------------------------------------------------------------------------------
    def albert(self, ids: Tensor) -> Tensor:
        t = ids.shape[0]
        E = "bert.embeddings."
        pos = self.per_t("pos", t, lambda: from_numpy(np.arange(t, dtype=np.int64), device="gpu", copy=True))
        zeros = self.per_t("zeros128", t, lambda: from_numpy(np.zeros((t, 128), np.float32), device="gpu", copy=True))
        e = ops.embedding2_add_f32_gpu(self.g(E + "word_embeddings.weight"), ids, self.g(E + "position_embeddings.weight"),
                                       pos)
        e = ops.add_bias_layernorm_f32_gpu(e, self.const("tt_row0", lambda: self.sd[E + "token_type_embeddings.weight"][0]),
                                           zeros, self.g(E + "LayerNorm.weight"), self.g(E + "LayerNorm.bias"), eps=1e-12)
        M = "bert.encoder.embedding_hidden_mapping_in"
        h = ops.gemm_bias_f32_gpu(e, self.g(M + ".weight", _t), self.g(M + ".bias"))
        L = "bert.encoder.albert_layer_groups.0.albert_layers.0."
        # the plain projections run as NT GEMMs on the [out, in] weights (the GEMM's B fragments are then 16-byte
        # runs of K); the result is the reference's x . W^T
        wqkv = self.const("albert#wqkv_nt", lambda: np.concatenate(
            [self.sd[L + f"attention.{n}.weight"] for n in ("query", "key", "value")], axis=0))
        bqkv = self.const("albert#bqkv", lambda: np.concatenate(
            [self.sd[L + f"attention.{n}.bias"] for n in ("query", "key", "value")]))
        # Below 64 output tiles (T <= 320) the projections feeding a LayerNorm split K over workgroups; their
        # partial planes then go straight into the LayerNorm, which sums them (add_bias_layernorm2_sk), instead of
        # through a reduction launch of their own (59 tokens: 24 launches fewer)
        sk = ops.splitk_planes(t, 768, 3) > 1

        def proj_ln(x, w, splits, b, g, beta):
            if sk:
                parts = ops.gemm_splitk_f32_gpu(x, self.g(w, _t), splits)
                return ops.add_bias_layernorm2_sk_f32_gpu(parts, self.g(b), h, self.g(g), self.g(beta), eps=1e-12)[1]
            return ops.add_bias_layernorm_f32_gpu(ops.gemm_nt_f32_gpu_mps(x, self.g(w)), self.g(b), h, self.g(g),
                                                  self.g(beta), eps=1e-12)

        for _ in range(12):
            a = ops.attention_qkv_sg_f32_gpu(ops.gemm_nt_f32_gpu_mps(h, wqkv), bqkv, heads=12)
            h = proj_ln(a, L + "attention.dense.weight", 3, L + "attention.dense.bias",
                        L + "attention.LayerNorm.weight", L + "attention.LayerNorm.bias")
            f = ops.gemm_steel_f32_gpu(h, self.g(L + "ffn.weight", _t), self.g(L + "ffn.bias"), act="gelu")
            h = proj_ln(f, L + "ffn_output.weight", 8, L + "ffn_output.bias", L + "full_layer_layer_norm.weight",
                        L + "full_layer_layer_norm.bias")
        return h

    def text_encoder_cnn(self, ids: Tensor) -> Tensor:
        """The TextEncoder up to its BiLSTM: embedding, 3 x (conv k5, LayerNorm, leaky 0.2) -> [T, 512]."""
        x = ops.embedding_f32_gpu(self.g("text_encoder.embedding.weight"), ids)  # [T, 512]
        for i in range(3):
            x = ops.conv1d_lc_f32_gpu(x, self.g(f"text_encoder.cnn.{i}.0.weight", _w_lc),
                                      self.g(f"text_encoder.cnn.{i}.0.bias"), padding=2)
            x = ops.layernorm_f32_gpu(x, self.g(f"text_encoder.cnn.{i}.1.gamma"), self.g(f"text_encoder.cnn.{i}.1.beta"),
                                      eps=1e-5)
            x = ops.leaky_lc_f32_gpu(x, 0.2)
        return x

    def _forward(self, ids: Tensor, ref_s: Tensor, dur: Tensor, noise: Tensor):
        frames = noise.shape[0] // 600
        s_d, s_p = ops.view(ref_s, [1, 128], 0), ops.view(ref_s, [1, 128], 128)
        bank_p = (ops.gemv4_f32_gpu(s_p, self.banks["predictor"][0], self.banks["predictor"][1]),
                  self.banks["predictor"][2])
        bank_d = (ops.gemv4_f32_gpu(s_d, self.banks["decoder"][0], self.banks["decoder"][1]), self.banks["decoder"][2])
        sp_vec = ops.view(s_p, [128])
        ctx = GpuContext.shared()
        # The TextEncoder (-> asr) depends only on the ids: it runs as a concurrent branch after ALBERT (which is on
        # the critical path and has the chip to itself; the reference overlaps it with GPU work the same way,
        # model.py:682-699). From 256 tokens on, its BiLSTM, of the same length as the duration encoder's first, runs
        # in the same recurrence launch (lstm2_bidir_t), so asr is ready long before the F0 / N curves the decoder
        # also needs, whatever order a graph runtime issues the branches in (487 tokens: 26.42 -> 26.25 ms). Below
        # that, waiting for the text encoder's convs before the first recurrence costs more than the shared launch
        # saves (59 tokens: 5.67 ms as a branch, 5.83 ms shared).
        bert = self.albert(ids)
        self._keep("bert", bert)
        shared = ids.shape[0] >= 256
        with ctx.branch(self.streams[0], 1):
            t_x = self.text_encoder_cnn(ids)
            if not shared:
                t_en = self.lstm(t_x, "text_encoder.lstm")
                asr = ops.repeat_interleave_f32_gpu(t_en, dur, frames)  # [F, 512] = asr^T
                self._keep("t_en", t_en)
        d_en = ops.gemm_bias_f32_gpu(bert, self.g("bert_encoder.weight", _t), self.g("bert_encoder.bias"))
        x = ops.concat_bcast_f32_gpu(d_en, sp_vec)
        if shared:
            ctx.join(self.streams[0])
            x, t_en = ops.lstm2_bidir_t_f32_gpu(x, *self.lstm_w("predictor.text_encoder.lstms.0"), t_x,
                                                *self.lstm_w("text_encoder.lstm"))
            with ctx.branch(self.streams[0], 1):
                asr = ops.repeat_interleave_f32_gpu(t_en, dur, frames)
                self._keep("t_en", t_en)
        for i in range(3):
            if i > 0 or not shared:
                x = self.lstm(x, f"predictor.text_encoder.lstms.{2 * i}")
            x = ops.adalayernorm_f32_gpu(x, self.style(bank_p, f"predictor.text_encoder.lstms.{2 * i + 1}.fc"))
            x = ops.concat_bcast_f32_gpu(x, sp_vec)
        self._keep("d", x)
        en = ops.repeat_interleave_f32_gpu(x, dur, frames)  # [F, 640]
        sh = self.lstm(en, "predictor.shared")  # [F, 512]

        def curve(name: str) -> Tensor:
            y = self.resblk(sh, bank_p, f"predictor.{name}.0", 512, 512, False)
            y = self.resblk(y, bank_p, f"predictor.{name}.1", 512, 256, True)
            y = self.resblk(y, bank_p, f"predictor.{name}.2", 256, 256, False)
            y = ops.gemv1_bias_f32_gpu(y, self.g(f"predictor.{name}_proj.weight", _col),
                                       self.g(f"predictor.{name}_proj.bias"))
            return ops.reshape(y, [2 * frames])

        # F0 and N are independent frame-rate conv stacks of a few hundred tiles each: run them side by side.
        with ctx.branch(self.streams[1], 2):
            n_curve = curve("N")
        f0 = curve("F0")
        # The generator's noise path (harmonic source -> STFT -> noise_convs.i -> noise_res.i) depends only on F0:
        # stage 0's block runs beside the decoder on one side stream, stage 1's on another, issued after the decoder
        # (below), that waits for the STFT; the generator joins each just before adding it.
        G = "decoder.generator."
        with ctx.branch(self.streams[2], 3):
            har_src = ops.harmonic_source_f32_gpu(f0, noise, self.g(G + "m_source.l_linear.weight", _flat),
                                                  self.g(G + "m_source.l_linear.bias"))
            har = ops.stft_magphase_lc_f32_gpu(har_src, 20, 5, cpad=32)  # [120 F + 1, 32]
            har_ready = ctx.mark(self.streams[2])
            self._keep("har_source", har_src)
            self._keep("har", har)
            xs_stage = [self.noise_block(har, bank_d, 0)]
        ctx.join(self.streams[1])
        ctx.join(self.streams[0])
        # decoder
        f0d = ops.conv1d_1ch_f32_gpu(f0, self.g("decoder.F0_conv.weight", _flat), self.g("decoder.F0_conv.bias"),
                                     stride=2, padding=1)
        nd = ops.conv1d_1ch_f32_gpu(n_curve, self.g("decoder.N_conv.weight", _flat), self.g("decoder.N_conv.bias"),
                                    stride=2, padding=1)
        fn_lc = ops.concat_pad_lc_f32_gpu(ops.reshape(f0d, [frames, 1]), ops.reshape(nd, [frames, 1]), cout=2)  # [F, 2]
        asr_res = ops.conv1d_lc_f32_gpu(asr, self.g("decoder.asr_res.0.weight", _w_lc), self.g("decoder.asr_res.0.bias"))
        extra = ops.concat_pad_lc_f32_gpu(asr_res, fn_lc, cout=66)  # [F, 66]
        x = self.resblk(ops.concat_pad_lc_f32_gpu(asr, fn_lc), bank_d, "decoder.encode", 514, 1024, False)
        for i in range(4):
            x = self.resblk(ops.concat_pad_lc_f32_gpu(x, extra), bank_d, f"decoder.decode.{i}", 1090,
                            1024 if i < 3 else 512, i == 3)
        self._keep("dec", x)
        # stage 1's noise block is issued after the decoder: beside it, its large stage-1-resolution convs slowed the
        # decoder's (the generator's stage 0 waits for the decoder, stage 1 only for this block): 28.11 -> 28.02 ms
        with ctx.branch(self.streams[3], 4):
            ctx.wait_mark(self.streams[3], har_ready)
            xs_stage.append(self.noise_block(har, bank_d, 1))
        # generator
        for i, (k_up, u) in enumerate(((20, 10), (12, 6))):
            x = ops.leaky_lc_f32_gpu(x, 0.1)
            y = ops.gemm_nt_f32_gpu_mps(x, self.g(G + f"ups.{i}.weight", _w_convt_nt))  # [Lin, K * Co]
            ctx.join(self.streams[2 + i])
            x = ops.convt_gather_lc_f32_gpu(y, self.g(G + f"ups.{i}.bias"), k_up, u, (k_up - u) // 2,
                                            add=xs_stage[i], reflect_left=(i == 1))
            xst = ops.channel_stats_lc_f32_gpu(x)  # shared by the three resblocks' first AdaIN
            # the three resblocks of a stage are independent: two run on side streams
            rb = [None, None, None]
            for j, kk in ((0, 3), (1, 7)):
                with ctx.branch(self.streams[j], 1 + j):
                    rb[j] = self.resblock1(x, bank_d, f"{G}resblocks.{3 * i + j}", kk, xst)
            rb[2] = self.resblock1(x, bank_d, f"{G}resblocks.{3 * i + 2}", 11, xst)
            ctx.join(self.streams[0])
            ctx.join(self.streams[1])
            self._keep(f"ups{i}", x)
            x = ops.add3_scale_f32_gpu(rb[0], rb[1], rb[2], 1.0 / 3.0)
            self._keep(f"stage{i}", x)
        ident = self.const("identity_affine128", lambda: np.stack([np.zeros(128), np.ones(128), np.zeros(128)]))
        # [120 F + 1, 64]: the 22 iSTFT logit columns, zero past them (output channels padded to a 64 block)
        post = self.conv(x, G + "conv_post", ident, 7, act="leaky", slope=0.01, co_pad=64)[0]
        audio = ops.istft_logits_lc_f32_gpu(post, n_fft=20, hop=5)
        return audio, f0, n_curve, post

    # ---- host API ----------------------------------------------------------------------------------------------
    def forward(self, ids, ref_s, dur, noise, inplace: bool = False):
        """One forward from host or device tensors; checks sum(dur) == F on the host (the reference's
        repeat_interleave reports a mismatch, kokoro_misc.cpp:253-260). Returns (audio, f0, n, post); post is
        f32[120 F + 1, 64]: the 22 iSTFT logit columns, then zeros."""
        dur_h = np.asarray(dur.numpy() if isinstance(dur, Tensor) else dur, np.int64)
        noise_rows = (noise.shape if isinstance(noise, Tensor) else np.shape(noise))[0]
        if noise_rows % 600 or int(dur_h.sum()) != noise_rows // 600 or (dur_h < 0).any():
            raise ValueError(f"durations sum to {int(dur_h.sum())} frames but the noise holds {noise_rows / 600} frames")
        args = [a if isinstance(a, Tensor) else from_numpy(np.ascontiguousarray(a), device="gpu", copy=True)
                for a in (ids, ref_s, dur, noise)]
        m = self.model if self.runtime == "capture" else self.compiled(args)
        return m.run_inplace(*args) if inplace else m(*args)

    def compiled(self, args):
        """The traced, compiled model of this input signature (built on first use)."""
        from .compiler import compile as lk_compile

        key = tuple(tuple(a.shape) for a in args)
        m = self._compiled.get(key)
        if m is None:
            m = lk_compile(self._forward, inputs=list(args), lanes=self.lanes)
            self._compiled[key] = m
        return m


def _t(a):
    return np.ascontiguousarray(a.T)


def _flat(a):
    return np.ascontiguousarray(a.reshape(-1))


def _col(a):  # [1, C, 1] projection -> [C, 1]
    return np.ascontiguousarray(a.reshape(-1, 1))


def _w_lc_32(a):  # noise convs: Ci = 22 padded to 32
    return _w_lc(a, 32)


def _pool_pad(a, cp):  # depthwise convT weight [C, 1, K] -> [Cpad, K]
    out = np.zeros((cp, a.shape[2]), np.float32)
    out[: a.shape[0]] = a[:, 0, :]
    return out
