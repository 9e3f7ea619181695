"""TEST INFRASTRUCTURE ONLY. numpy restatement of the reference's f16 Qwen3(-ASR) LM ops and of its "basic" graph
(models/qwen3_asr/model.py:275-292; op contracts python/lokinfer/ops/f16.py; host kernels kernels/cpu/f16_basic.cpp
in lariaus/lokinfer): f16 storage, math in `dt` (float64 for the per-op checks, as the reference's kernel tests
compose in float64; float32 for the whole model, the contract's own arithmetic), one rounding to f16 at every op's
output. With rounding off (`Ops(dt, rounding=False)`) the graph is the plain float model, which the tests pin
against transformers' Qwen3ForCausalLM.
"""
from __future__ import annotations

import numpy as np

PAD_ID = 151676


def inv_freq(theta: float) -> np.ndarray:
    """f32 inv_freq[j] = 1 / powf(theta, 2j / 128) with the C library's powf, as the reference's host kernel computes
    it (std::pow(float, float), kernels/cpu/f16_basic.cpp:262-263); numpy's float32 power may use another
    implementation and differ in the last bit, which moves an angle p inv_freq by p ulps."""
    import ctypes
    import ctypes.util

    libm = ctypes.CDLL(ctypes.util.find_library("m"))
    libm.powf.restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    return np.array([np.float32(1) / np.float32(libm.powf(np.float32(theta), np.float32(2 * j) / np.float32(128)))
                     for j in range(64)], np.float32)


class Ops:
    def __init__(self, dt=np.float64, rounding: bool = True):
        self.dt, self.rounding = dt, rounding

    def r16(self, x):
        x = np.asarray(x, self.dt)
        return x.astype(np.float16).astype(self.dt) if self.rounding else x

    def c(self, x):
        return np.asarray(x, self.dt)

    # f16_basic.cpp:424-434 gemm (f32 accumulation, one rounding)
    def gemm(self, x, w):
        return self.r16(self.c(x) @ self.c(w))

    def add(self, x, y):
        return self.r16(self.c(x) + self.c(y))

    def silu_mul(self, g, u):
        g, u = self.c(g), self.c(u)
        return self.r16(g / (1 + np.exp(-g)) * u)

    # f16_basic.cpp:215-243: h = f16(x r), y = f16(g h), r = 1 / sqrt(mean(x^2) + eps)
    def rmsnorm(self, x, g, eps=1e-6, width=None):
        x = self.c(x)
        shp = x.shape
        w = shp[-1] if width is None else width
        xg = x.reshape(-1, w)
        r = 1 / np.sqrt((xg * xg).sum(-1, keepdims=True) / w + eps)
        h = self.r16(xg * r)
        return self.r16(self.c(g) * h).reshape(shp)

    def rmsnorm_heads(self, x, g, eps=1e-6):
        return self.rmsnorm(x, g, eps, width=len(g))

    # f16_basic.cpp:248-283: inv_freq[j] = f32(1 / f32(theta^(2j/128))), angle = f32(f32(p) inv_freq[j]), cos / sin of
    # that angle evaluated in double and rounded to f32; the rotation in `dt`
    def rope(self, x, pos, theta=1e6):
        x = self.c(x)
        t, c = x.shape
        invf = inv_freq(theta)
        p = (pos + np.arange(t)).astype(np.float32)
        ang = (p[:, None] * invf[None, :]).astype(np.float32)
        cs = np.cos(ang.astype(np.float64)).astype(np.float32).astype(self.dt)
        sn = np.sin(ang.astype(np.float64)).astype(np.float32).astype(self.dt)
        out = np.empty_like(x)
        for h0 in range(0, c, 128):
            lo, hi = x[:, h0:h0 + 64], x[:, h0 + 64:h0 + 128]
            out[:, h0:h0 + 64] = lo * cs - hi * sn
            out[:, h0 + 64:h0 + 128] = hi * cs + lo * sn
        return self.r16(out)

    def embedding(self, ids, table):
        ids = np.asarray(ids)
        if (ids < 0).any() or (ids >= len(table)).any():
            raise ValueError("embedding: token id out of range")
        return self.c(table[ids])

    # f16_basic.cpp:327-345
    def scatter_audio(self, x, ids, audio, pad_id=PAD_ID):
        x = self.c(x).copy()
        pads = np.nonzero(np.asarray(ids) == pad_id)[0]
        if len(pads) > len(audio):
            raise ValueError("scatter_audio: more audio pad ids than audio rows")
        x[pads] = self.c(audio)[:len(pads)]
        return x

    # f16_basic.cpp:409-440: query i (position pos + i) of q-head h attends to cache rows 0 .. pos + i of kv-head
    # h / (q_heads / kv_heads), scale 1 / sqrt(hd), output rounded once
    def attention_gqa(self, q, kc, vc, pos, q_heads, kv_heads):
        q, kc, vc = self.c(q), self.c(kc), self.c(vc)
        t = q.shape[0]
        hd = q.shape[1] // q_heads
        if pos < 0 or pos + t > kc.shape[0]:
            raise ValueError("attention_gqa: pos + T exceeds the cache")
        out = np.zeros_like(q)
        grp = q_heads // kv_heads
        for h in range(q_heads):
            ko = (h // grp) * hd
            K, V = kc[:pos + t, ko:ko + hd], vc[:pos + t, ko:ko + hd]
            s = q[:, h * hd:(h + 1) * hd] @ K.T / np.sqrt(hd)
            s = np.where(np.arange(pos + t)[None, :] <= (pos + np.arange(t))[:, None], s, -np.inf)
            s = np.exp(s - s.max(-1, keepdims=True))
            out[:, h * hd:(h + 1) * hd] = (s / s.sum(-1, keepdims=True)) @ V
        return self.r16(out)

    def lm_head_last(self, x, table):
        return self.c(x)[-1:] @ self.c(table).T


class OracleLm:
    """The basic graph over numpy caches f16-valued in `dt` (reference build_generate, model.py:237-292)."""

    def __init__(self, sd, cfg, ops: Ops, capacity: int):
        self.sd, self.cfg, self.o = sd, cfg, ops
        self.kv = np.zeros((cfg.layers, 2, capacity, cfg.dk), ops.dt)
        self._w = {}

    def w(self, key):
        if key not in self._w:
            self._w[key] = self.o.c(self.sd[key])
        return self._w[key]

    def __call__(self, ids, audio, pos, return_hidden=False):
        o, c = self.o, self.cfg
        ids = np.asarray(ids, np.int64)
        t = len(ids)
        h = o.scatter_audio(o.embedding(ids, self.sd["embed"]), ids, audio)
        for i in range(c.layers):
            p = f"lm.{i}."
            a = o.rmsnorm(h, self.w(p + "ln1.g"), c.eps)
            q = o.rope(o.rmsnorm_heads(o.gemm(a, self.w(p + "q.w")), self.w(p + "qn.g"), c.eps), pos, c.theta)
            k = o.rope(o.rmsnorm_heads(o.gemm(a, self.w(p + "k.w")), self.w(p + "kn.g"), c.eps), pos, c.theta)
            v = o.gemm(a, self.w(p + "v.w"))
            if pos + t > self.kv.shape[2]:
                raise ValueError("kv_write: pos + T exceeds the cache")
            self.kv[i, 0, pos:pos + t] = k
            self.kv[i, 1, pos:pos + t] = v
            att = o.attention_gqa(q, self.kv[i, 0], self.kv[i, 1], pos, c.qh, c.kvh)
            h = o.add(h, o.gemm(att, self.w(p + "o.w")))
            a = o.rmsnorm(h, self.w(p + "ln2.g"), c.eps)
            h = o.add(h, o.gemm(o.silu_mul(o.gemm(a, self.w(p + "gate.w")), o.gemm(a, self.w(p + "up.w"))),
                                self.w(p + "down.w")))
        normed = o.rmsnorm(h, self.w("lm.norm.g"), c.eps)
        logits = o.lm_head_last(normed, self.w("embed"))
        return (logits, normed) if return_hidden else logits


def hf_model(sd, cfg):
    """transformers Qwen3ForCausalLM (built locally, float64) loaded with the folded weights (linear weights
    transposed back to [out, in], the tied head from "embed")."""
    import torch
    from transformers import Qwen3Config, Qwen3ForCausalLM

    hc = Qwen3Config(vocab_size=cfg.vocab, hidden_size=cfg.d, intermediate_size=cfg.ffn,
                     num_hidden_layers=cfg.layers, num_attention_heads=cfg.qh, num_key_value_heads=cfg.kvh,
                     head_dim=cfg.hd, rms_norm_eps=cfg.eps, rope_theta=cfg.theta, tie_word_embeddings=True,
                     attention_bias=False, max_position_embeddings=4096)
    hc._attn_implementation = "eager"
    m = Qwen3ForCausalLM(hc).eval().to(torch.float64)
    T = lambda a: torch.from_numpy(np.asarray(a, np.float64))  # noqa: E731
    st = {"model.embed_tokens.weight": T(sd["embed"]), "model.norm.weight": T(sd["lm.norm.g"]),
          "lm_head.weight": T(sd["embed"])}
    for i in range(cfg.layers):
        p, L = f"lm.{i}.", f"model.layers.{i}."
        st[L + "input_layernorm.weight"] = T(sd[p + "ln1.g"])
        st[L + "post_attention_layernorm.weight"] = T(sd[p + "ln2.g"])
        for n, hfn in (("q", "q_proj"), ("k", "k_proj"), ("v", "v_proj"), ("o", "o_proj")):
            st[L + f"self_attn.{hfn}.weight"] = T(sd[p + n + ".w"]).T.contiguous()
        st[L + "self_attn.q_norm.weight"] = T(sd[p + "qn.g"])
        st[L + "self_attn.k_norm.weight"] = T(sd[p + "kn.g"])
        for n, hfn in (("gate", "gate_proj"), ("up", "up_proj"), ("down", "down_proj")):
            st[L + f"mlp.{hfn}.weight"] = T(sd[p + n + ".w"]).T.contiguous()
    missing, unexpected = m.load_state_dict(st, strict=False)
    assert not unexpected and all("rotary" in k for k in missing), (missing, unexpected)
    return m
