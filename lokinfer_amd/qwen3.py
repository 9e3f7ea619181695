"""The Qwen3-ASR language model (f16) on the MI355X kernels: the reference's `build_generate`
(models/qwen3_asr/model.py:237-294, the "opt" layer :393-401 in lariaus/lokinfer) and its caller loop
(`transcribe`, :309-336).

A call takes ids i64[T] (T new tokens), audio f16[A, D] (the rows the chunk's <|audio_pad|> ids take, in order; any
one row when there are none), pos (tokens already in the cache) and the caller-owned MUTABLE KV cache
kv f16[L, 2, P, kvh 128] (written in place), and returns the logits f32[1, V] of the last new token. Prefill chunks
and decode steps are the same call; one compiled graph per (T, A, P) signature (decode steps replay one graph).

Per layer (variant "opt", the reference's _lm_layer_opt; at T = 1 two fusions of its ops, `_layer_decode`):
  qkv = rmsnorm_gemm_opt(h, ln1, [q|k|v])                      M = 1: one GEMV that normalizes the row itself
  q   = qknorm_rope_kv_opt(qkv, qn, kn, pos, kc, vc)            QK-norm + RoPE, k and v written to the cache
  att = attention_gqa_opt(q, kc, vc, pos)                       causal GQA 16 / 8 heads x 128
  h   = gemm_add_opt(att, o, h)
  m   = rmsnorm_gemm_swiglu_opt(h, ln2, [gate|up])
  h   = gemm_add_opt(m, down, h)
then logits = lm_head_last(rmsnorm(h, norm), embed). Variant "basic" is the reference's op-per-op graph
(:275-287). Weights are the reference's folded layout (`fold_weights`, :19-66: linear weights [in, out], the tied
embedding stored once as "embed"), packed on upload as W^T for the kernels.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from . import ops
from . import f16_gpu as F
from .compiler import capture as lk_capture
from .runtime import GpuContext
from .tensor import Tensor, f16


@dataclass(frozen=True)
class Qwen3Config:
    """LM hyper-parameters (reference model.py:12-13: 28 layers, hidden 2048, GQA 16 / 8 x 128, SwiGLU 6144,
    vocab 151936, RoPE theta 1e6, RMSNorm eps 1e-6)."""
    layers: int = 28
    d: int = 2048
    qh: int = 16
    kvh: int = 8
    hd: int = 128
    ffn: int = 6144
    vocab: int = 151936
    theta: float = 1e6
    eps: float = 1e-6

    @property
    def dq(self) -> int:
        return self.qh * self.hd

    @property
    def dk(self) -> int:
        return self.kvh * self.hd


CONFIG5 = Qwen3Config()
AUDIO_START = 9  # the <|audio_pad|> run starts after the 9 prefix ids (reference model.py:301)
EOS = (151643, 151645)


def param_shapes(cfg: Qwen3Config = CONFIG5) -> dict[str, tuple]:
    """The reference's folded LM parameter names and shapes (model.py:55-66)."""
    s = {"embed": (cfg.vocab, cfg.d), "lm.norm.g": (cfg.d,)}
    for i in range(cfg.layers):
        p = f"lm.{i}."
        s.update({p + "ln1.g": (cfg.d,), p + "ln2.g": (cfg.d,), p + "q.w": (cfg.d, cfg.dq), p + "k.w": (cfg.d, cfg.dk),
                  p + "v.w": (cfg.d, cfg.dk), p + "o.w": (cfg.dq, cfg.d), p + "qn.g": (cfg.hd,), p + "kn.g": (cfg.hd,),
                  p + "gate.w": (cfg.d, cfg.ffn), p + "up.w": (cfg.d, cfg.ffn), p + "down.w": (cfg.ffn, cfg.d)})
    return s


def random_weights(cfg: Qwen3Config = CONFIG5, seed: int = 2025) -> dict[str, np.ndarray]:
    """Random-init f16 weights: every parameter ~ N(0, 0.02) (numpy default_rng(seed + index) over the sorted names),
    RMSNorm gains 1 + N(0, 0.02) so that every term of the norm is exercised."""
    sd = {}
    for i, (k, shape) in enumerate(sorted(param_shapes(cfg).items())):
        a = np.random.default_rng(seed + i).standard_normal(shape, dtype=np.float32) * np.float32(0.02)
        if k.endswith(".g"):
            a += np.float32(1.0)
        sd[k] = a.astype(np.float16)
    return sd


def config5_inputs(cfg: Qwen3Config = CONFIG5, n_audio: int = 400, n_prompt: int = 16, seed: int = 77):
    """Config 5's prefill: 9 seeded prefix ids, n_audio <|audio_pad|> ids, the other n_prompt - 9 seeded ids; audio
    rows ~ N(0, 1) f16[n_audio, D]."""
    r = np.random.default_rng(seed)
    pre = r.integers(0, min(cfg.vocab, F.PAD_ID), AUDIO_START)
    post = r.integers(0, min(cfg.vocab, F.PAD_ID), n_prompt - AUDIO_START)
    ids = np.concatenate([pre, np.full(n_audio, F.PAD_ID), post]).astype(np.int64)
    audio = r.standard_normal((n_audio, cfg.d), dtype=np.float32).astype(np.float16)
    return ids, audio


class Qwen3Lm:
    """Weights uploaded and packed once; call(ids, audio, pos, kv) -> logits (reference build_generate)."""

    def __init__(self, sd: dict[str, np.ndarray], cfg: Qwen3Config = CONFIG5, variant: str = "opt",
                 graph: bool = True):
        if variant not in ("basic", "opt"):
            raise ValueError(f"variant {variant!r}: expected 'basic' or 'opt'")
        self.cfg, self.variant = cfg, variant
        dev = GpuContext.shared().device
        self.device = dev

        def up(a):
            return Tensor(torch.from_numpy(np.ascontiguousarray(a, np.float16)).to(dev))

        self.embed = up(sd["embed"])
        self.norm = up(sd["lm.norm.g"])
        self.layers = []
        for i in range(cfg.layers):
            p = f"lm.{i}."
            L = {k: up(sd[p + k]) for k in ("ln1.g", "ln2.g", "qn.g", "kn.g")}
            if variant == "opt":  # the reference's fold_opt concatenations (model.py:349-368)
                L["qkv"] = F.pack(np.concatenate([sd[p + "q.w"], sd[p + "k.w"], sd[p + "v.w"]], axis=1))
                L["gateup"] = F.pack(np.concatenate([sd[p + "gate.w"], sd[p + "up.w"]], axis=1))
            else:
                for k in ("q", "k", "v", "gate", "up"):
                    L[k] = F.pack(sd[p + k + ".w"])
            L["o"] = F.pack(sd[p + "o.w"])
            L["down"] = F.pack(sd[p + "down.w"])
            self.layers.append(L)
        self.positions = torch.arange(1 << 16, dtype=torch.int64, device=dev)  # device pos views, no host copies
        self.counters = Tensor(torch.zeros(cfg.qh, dtype=torch.int32, device=dev))  # decode attention merge counters
        self.model = lk_capture(self._fn, graph=graph, mutable=(3,))  # kv: the caller's cache, written in place

    def kv_cache(self, capacity: int) -> Tensor:
        """A zeroed cache for `capacity` positions: f16[L, 2, capacity, kvh 128] on the device (reference kv_cache,
        model.py:295-305)."""
        c = self.cfg
        return Tensor(torch.zeros(c.layers, 2, capacity, c.dk, dtype=torch.float16, device=self.device))

    def _layer_opt(self, L, h, pos, kc, vc):
        c = self.cfg
        qkv, _ = F.rmsnorm_gemm_opt_f16_gpu(h, L["ln1.g"], L["qkv"], c.eps)
        q = F.qknorm_rope_kv_opt_f16_gpu(qkv, L["qn.g"], L["kn.g"], pos, kc, vc, c.eps, c.theta)
        att = F.attention_gqa_opt_f16_gpu(q, kc, vc, pos, q_heads=c.qh, kv_heads=c.kvh)
        h = F.gemm_add_opt_f16_gpu(att, L["o"], h)
        m, _ = F.rmsnorm_gemm_swiglu_opt_f16_gpu(h, L["ln2.g"], L["gateup"], c.eps)
        return F.gemm_add_opt_f16_gpu(m, L["down"], h)

    def _layer_basic(self, L, h, pos, kc, vc):
        c = self.cfg
        a = F.rmsnorm_f16_gpu(h, L["ln1.g"], c.eps)
        q = F.rope_f16_gpu(F.rmsnorm_heads_f16_gpu(F.gemm_f16_gpu(a, L["q"]), L["qn.g"], c.eps), pos, c.theta)
        k = F.rope_f16_gpu(F.rmsnorm_heads_f16_gpu(F.gemm_f16_gpu(a, L["k"]), L["kn.g"], c.eps), pos, c.theta)
        F.kv_write_f16_gpu(kc, vc, k, F.gemm_f16_gpu(a, L["v"]), pos)
        att = F.attention_gqa_f16_gpu(q, kc, vc, pos, q_heads=c.qh, kv_heads=c.kvh)
        h = F.add_f16_gpu(h, F.gemm_f16_gpu(att, L["o"]))
        a = F.rmsnorm_f16_gpu(h, L["ln2.g"], c.eps)
        g = F.silu_mul_f16_gpu(F.gemm_f16_gpu(a, L["gate"]), F.gemm_f16_gpu(a, L["up"]))
        return F.add_f16_gpu(h, F.gemm_f16_gpu(g, L["down"]))

    def _layer_decode(self, L, h, pos, kc, vc):
        """The opt layer at T = 1 in 5 launches: QK-norm / RoPE / KV write, the key-split attention and its merge in
        one (equal to qknorm_rope_kv_opt + attention_gqa_opt bit for bit)."""
        c = self.cfg
        qkv, _ = F.rmsnorm_gemm_opt_f16_gpu(h, L["ln1.g"], L["qkv"], c.eps)
        att = F.attention_decode_qkr_opt_f16_gpu(qkv, L["qn.g"], L["kn.g"], pos, kc, vc, self.counters, c.eps, c.theta)
        h = F.gemm_add_opt_f16_gpu(att, L["o"], h)
        m, _ = F.rmsnorm_gemm_swiglu_opt_f16_gpu(h, L["ln2.g"], L["gateup"], c.eps)
        return F.gemm_add_opt_f16_gpu(m, L["down"], h)

    def _fn(self, ids: Tensor, audio: Tensor, pos: Tensor, kv: Tensor):
        c = self.cfg
        h = F.scatter_audio_f16_gpu(F.embedding_f16_gpu(ids, self.embed), ids, audio)
        opt = self.variant == "opt"
        layer = self._layer_basic
        if opt:
            layer = self._layer_decode if ids.shape[0] == 1 else self._layer_opt
        for i, L in enumerate(self.layers):
            kc, vc = Tensor(kv.t[i, 0]), Tensor(kv.t[i, 1])  # views of the caller's cache
            h = layer(L, h, pos, kc, vc)
        if opt:
            logits = F.rmsnorm_lm_head_last_opt_f16_gpu(h, self.norm, self.embed, c.eps)
        else:
            logits = F.lm_head_last_f16_gpu(F.rmsnorm_f16_gpu(h, self.norm, c.eps), self.embed)
        return logits, ops.argmax_f32_gpu(logits)

    def run(self, ids, audio, pos: int, kv: Tensor):
        """(logits f32[1, V], argmax i64[1]) of the last new token; the compiled graph's own buffers (overwritten by
        the next call with the same shapes). pos + T must fit the cache."""
        c = self.cfg
        ids = self._dev(ids, np.int64)
        audio = self._dev(audio, np.float16)
        T, P = ids.shape[0], kv.shape[2]
        if tuple(kv.shape) != (c.layers, 2, P, c.dk) or kv.dtype != f16:
            raise ValueError(f"kv must be f16[{c.layers}, 2, P, {c.dk}]")
        if not (T >= 1 and 0 <= pos and pos + T <= P):
            raise ValueError(f"qwen3: positions {pos}..{pos + T - 1} outside the {P}-row cache")
        p = Tensor(self.positions[pos:pos + 1] if pos < self.positions.numel()
                   else torch.tensor([pos], dtype=torch.int64, device=self.device))
        return self.model.run_inplace(ids, audio, p, kv)

    def __call__(self, ids, audio, pos: int, kv: Tensor) -> np.ndarray:
        """Reference model(ids, audio, pos, kv): logits f32[1, V] (a host copy)."""
        return self.run(ids, audio, pos, kv)[0].numpy()

    def _dev(self, x, dtype) -> Tensor:
        if isinstance(x, Tensor):
            return x if x.device == "gpu" else Tensor(x.t.to(self.device))
        return Tensor(torch.from_numpy(np.ascontiguousarray(x, dtype)).to(self.device))


def transcribe(model: Qwen3Lm, ids: np.ndarray, audio: np.ndarray, max_new: int, chunk: int = 2048,
               kv: Tensor | None = None, stop_at_eos: bool = True) -> list[int]:
    """The reference's caller loop (model.py:309-336) for the LM: prefill in chunks of <= `chunk` ids (each chunk
    gets the audio rows its pad ids take), then greedy decode until eos or max_new tokens. Each step's argmax stays
    on the device and feeds the next step; the tokens come back once at the end (an eos check reads one token per
    step only when stop_at_eos is set)."""
    c = model.cfg
    T = len(ids)
    if kv is None:
        kv = model.kv_cache(T + max_new)
    n_audio = len(audio)
    dummy = np.zeros((1, c.d), np.float16)
    am = None
    for s in range(0, T, chunk):
        e = min(T, s + chunk)
        k0, k1 = min(max(s - AUDIO_START, 0), n_audio), min(max(e - AUDIO_START, 0), n_audio)
        rows = audio[k0:k1] if k1 > k0 else dummy
        _, am = model.run(ids[s:e], rows, s, kv)
    toks = torch.empty(max_new, dtype=torch.int64, device=model.device)
    dummy_t = model._dev(dummy, np.float16)
    pos, n = T, 0
    while n < max_new:
        toks[n:n + 1].copy_(am.t)
        n += 1
        if n >= max_new or (stop_at_eos and int(toks[n - 1]) in EOS):
            break
        _, am = model.run(Tensor(toks[n - 1:n]), dummy_t, pos, kv)
        pos += 1
    return [int(v) for v in toks[:n].cpu()]
