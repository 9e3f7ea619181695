"""GPT-2 124M decode step on the MI355X kernels: the graph of the reference's `build_decode(sd, device="gpu")`
(models/gpt2.py:161-249 in lariaus/lokinfer), GPU-resident end to end.

Per step (inputs tok i64[1], pos i64[1], both on the device):
  h = wte[tok] + wpe[pos];  ln = LN_1(h)
  per layer: qkv = gemv4(ln, c_attn.W) -> attention_decode_split (writes k, v + bias at row pos of the layer's
             persistent [1024, 768] caches, attends over rows 0..pos) -> gemv4(., c_proj.W) ->
             (h, ln) = add_bias_layernorm2(., c_proj.b, h, LN_2) -> gemv4_bias_gelu(ln, c_fc) -> gemv4(., mlp.c_proj.W)
             -> (h, ln) = add_bias_layernorm2(., mlp.c_proj.b, h, next LN_1 or ln_f)
  logits = ln . wte^T (tied LM head, gemm_nt);  next = argmax(logits) on the device
The reference does the two embedding lookups on the CPU and the argmax in Python; here they are device kernels
so a step is one captured HIP graph.

Gpt2Generator is the reference's `build_generate` (models/gpt2.py:250-333): chunked prefill and decode over the same
persistent caches. A call with T new tokens at start position pos returns the logits of the last one; T = 1 runs the
decode step above, T > 1 the chunk forward (GEMM, kv_write_rows + flash attention over the cache, split-K
projections into bias + residual + LayerNorm).

By default (fused=True) each layer runs the same arithmetic in 5 launches instead of 13: the GEMVs write
row-slice partial sums and the consumer of each GEMV sums the slices itself (the decode-attention chunk kernel
for qkv; the next partial GEMV for the attention merge, for gelu(c_fc) and for bias + residual + LayerNorm, the
new residual stream written by one of its workgroups). The embedding lookups and LN_1 of layer 0 open the first
partial GEMV, and ln_f, the LM head and the argmax are one op (a row-dot pass that also leaves per-workgroup
(max, index) pairs, then a one-workgroup pass over the pairs): 62 launches per step. fused=False keeps the
reference's op sequence.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops
from .compiler import capture as lk_capture
from .tensor import Tensor, from_numpy

N_LAYER, D, HEADS, N_POS, VOCAB, FFN = 12, 768, 12, 1024, 50257, 3072
LN_EPS = 1e-5


def param_shapes() -> dict[str, tuple]:
    """HF GPT2LMHeadModel parameter names and shapes (Conv1D weights are [in, out])."""
    s = {"transformer.wte.weight": (VOCAB, D), "transformer.wpe.weight": (N_POS, D),
         "transformer.ln_f.weight": (D,), "transformer.ln_f.bias": (D,)}
    for i in range(N_LAYER):
        L = f"transformer.h.{i}."
        s.update({L + "ln_1.weight": (D,), L + "ln_1.bias": (D,), L + "attn.c_attn.weight": (D, 3 * D),
                  L + "attn.c_attn.bias": (3 * D,), L + "attn.c_proj.weight": (D, D), L + "attn.c_proj.bias": (D,),
                  L + "ln_2.weight": (D,), L + "ln_2.bias": (D,), L + "mlp.c_fc.weight": (D, FFN),
                  L + "mlp.c_fc.bias": (FFN,), L + "mlp.c_proj.weight": (FFN, D), L + "mlp.c_proj.bias": (D,)})
    return s


def random_weights(seed: int = 2024) -> dict[str, np.ndarray]:
    """Random-init state dict: every parameter ~ N(0, 0.02) (numpy default_rng(seed + index) over the sorted
    names), LayerNorm weights 1 + N(0, 0.02) so that every term of the LN is exercised."""
    sd = {}
    for i, (k, shape) in enumerate(sorted(param_shapes().items())):
        a = np.random.default_rng(seed + i).standard_normal(shape).astype(np.float32) * np.float32(0.02)
        if k.endswith(("ln_1.weight", "ln_2.weight", "ln_f.weight")):
            a = a + np.float32(1.0)
        sd[k] = a.astype(np.float32)
    return sd


class Gpt2Decoder:
    """Weights uploaded once; 12 persistent K/V caches f32[1024, 768] on the device (the reference's
    lk.persistent_buffer caches, models/gpt2.py:186-188)."""

    def __init__(self, sd: dict[str, np.ndarray], graph: bool = True, fused: bool = True):
        self.w = {k: from_numpy(v, device="gpu", copy=True) for k, v in sd.items()}
        dev = self.w["transformer.wte.weight"].t.device
        self.caches = [(Tensor(torch.zeros(N_POS, D, device=dev)), Tensor(torch.zeros(N_POS, D, device=dev)))
                       for _ in range(N_LAYER)]
        self.fused = fused
        # the step graph reads tok and pos from these two buffers in place (a caller that writes them itself, as
        # a serving loop does, replays with no input copy)
        self.tok = Tensor(torch.zeros(1, dtype=torch.int64, device=dev))
        self.pos = Tensor(torch.zeros(1, dtype=torch.int64, device=dev))
        self.step_model = lk_capture(self._step, graph=graph, by_ref=(0, 1))

    def _step(self, tok: Tensor, pos: Tensor):
        w = self.w
        P = "transformer."
        if self.fused:
            # 5 launches per layer: each GEMV writes row-slice partial sums and its consumer reduces them (the
            # decode-attention chunk kernel for qkv, the next partial GEMV for the attention merge, for gelu(c_fc)
            # and for bias + residual + LayerNorm); the embedding lookups open the first GEMV, and the last
            # LayerNorm and the argmax are folded into the LM head
            qp, h = ops.gemv_partial_embed_ln_f32_gpu(w[P + "wte.weight"], tok, w[P + "wpe.weight"], pos,
                                                      w[P + "h.0.ln_1.weight"], w[P + "h.0.ln_1.bias"],
                                                      w[P + "h.0.attn.c_attn.weight"], eps=LN_EPS)
            for i, (kc, vc) in enumerate(self.caches):
                L = f"{P}h.{i}."
                ch = ops.attention_decode_part_f32_gpu(qp, kc, vc, pos, w[L + "attn.c_attn.bias"], heads=HEADS)
                op = ops.gemv_partial_attn_f32_gpu(ch, w[L + "attn.c_proj.weight"])
                fp, h = ops.gemv_partial_res_ln_f32_gpu(op, w[L + "attn.c_proj.bias"], h, w[L + "ln_2.weight"],
                                                        w[L + "ln_2.bias"], w[L + "mlp.c_fc.weight"], eps=LN_EPS)
                mp = ops.gemv_partial_gelu_f32_gpu(fp, w[L + "mlp.c_fc.bias"], w[L + "mlp.c_proj.weight"])
                if i + 1 < N_LAYER:
                    N = f"{P}h.{i + 1}."
                    qp, h = ops.gemv_partial_res_ln_f32_gpu(mp, w[L + "mlp.c_proj.bias"], h, w[N + "ln_1.weight"],
                                                            w[N + "ln_1.bias"], w[N + "attn.c_attn.weight"],
                                                            eps=LN_EPS)
                else:
                    return ops.lm_head_ln_argmax_f32_gpu(mp, w[L + "mlp.c_proj.bias"], h, w[P + "ln_f.weight"],
                                                         w[P + "ln_f.bias"], w[P + "wte.weight"], eps=LN_EPS)
        h = ops.embedding2_add_f32_gpu(w[P + "wte.weight"], tok, w[P + "wpe.weight"], pos)
        ln = ops.layernorm_f32_gpu(h, w[P + "h.0.ln_1.weight"], w[P + "h.0.ln_1.bias"], eps=LN_EPS)
        for i, (kc, vc) in enumerate(self.caches):
            L = f"{P}h.{i}."
            nxt = f"{P}h.{i + 1}.ln_1." if i + 1 < N_LAYER else P + "ln_f."
            qkv = ops.gemv4_f32_gpu(ln, w[L + "attn.c_attn.weight"])
            att = ops.attention_decode_split_f32_gpu(qkv, kc, vc, pos, w[L + "attn.c_attn.bias"], heads=HEADS)
            o = ops.gemv4_f32_gpu(att, w[L + "attn.c_proj.weight"])
            h, ln = ops.add_bias_layernorm2_f32_gpu(o, w[L + "attn.c_proj.bias"], h, w[L + "ln_2.weight"],
                                                    w[L + "ln_2.bias"], eps=LN_EPS)
            f = ops.gemv4_f32_gpu(ln, w[L + "mlp.c_fc.weight"], w[L + "mlp.c_fc.bias"], act="gelu")
            o = ops.gemv4_f32_gpu(f, w[L + "mlp.c_proj.weight"])
            h, ln = ops.add_bias_layernorm2_f32_gpu(o, w[L + "mlp.c_proj.bias"], h, w[nxt + "weight"], w[nxt + "bias"],
                                                    eps=LN_EPS)
        logits = ops.gemm_nt_f32_gpu_mps(ln, w[P + "wte.weight"])
        return logits, ops.argmax_f32_gpu(logits)

    def step(self, tok: Tensor, pos: Tensor):
        """One decode step; returns (logits f32[1, 50257], argmax i64[1]) as the graph's output buffers
        (overwritten by the next step). tok and pos are copied into self.tok / self.pos unless they are those
        buffers."""
        for src, dst in ((tok, self.tok), (pos, self.pos)):
            if src.t.data_ptr() != dst.t.data_ptr():
                dst.t.copy_(src.t.reshape(1))
        return self.step_model.run_inplace(self.tok, self.pos)

    def prefill(self, ids: np.ndarray) -> None:
        """Fills the caches by stepping the prompt tokens at positions 0..len-1."""
        dev = self.w["transformer.wte.weight"].t.device
        for p, t in enumerate(np.asarray(ids, np.int64)):
            self.step(Tensor(torch.tensor([int(t)], device=dev)), Tensor(torch.tensor([p], device=dev)))


class Gpt2Generator(Gpt2Decoder):
    """Chunked prefill + decode sharing the caches (reference build_generate, models/gpt2.py:250-333). sk: split-K
    factors of the two N = 768 projections for T > 1 ((0, 0) = plain GEMM + add_bias_layernorm2). chunk_graph:
    capture each chunk length's forward as a HIP graph (pays off when one length recurs; a one-off prompt runs
    eagerly)."""

    def __init__(self, sd: dict[str, np.ndarray], graph: bool = True, fused: bool = True, sk=(2, 4),
                 chunk_graph: bool = False):
        super().__init__(sd, graph=graph, fused=fused)
        self.sk = tuple(sk)
        dev = self.w["transformer.wte.weight"].t.device
        self.positions = torch.arange(N_POS, dtype=torch.int64, device=dev)  # device pos views, no host copies
        self.chunk_model = lk_capture(self._chunk, graph=chunk_graph)

    def _chunk(self, ids: Tensor, pos: Tensor):
        w = self.w
        P = "transformer."
        T = ids.shape[0]
        pids = ops.arange_offset_i64_gpu(pos, T)
        h = ops.embedding2_add_f32_gpu(w[P + "wte.weight"], ids, w[P + "wpe.weight"], pids)
        ln = ops.layernorm_f32_gpu(h, w[P + "h.0.ln_1.weight"], w[P + "h.0.ln_1.bias"], eps=LN_EPS)

        def proj_ln(x, wk, res, ln_key, splits):  # (res + x @ W + b, LN of it)
            if splits:
                parts = ops.gemm_auto_sk_f32_gpu(x, w[wk + "weight"], splits)
                return ops.add_bias_layernorm2_sk_f32_gpu(parts, w[wk + "bias"], res, w[ln_key + "weight"],
                                                          w[ln_key + "bias"], eps=LN_EPS)
            return ops.add_bias_layernorm2_f32_gpu(ops.gemm_auto_f32_gpu(x, w[wk + "weight"]), w[wk + "bias"], res,
                                                   w[ln_key + "weight"], w[ln_key + "bias"], eps=LN_EPS)

        for i, (kc, vc) in enumerate(self.caches):
            L = f"{P}h.{i}."
            nxt = f"{P}h.{i + 1}.ln_1." if i + 1 < N_LAYER else P + "ln_f."
            qkv = ops.gemm_auto_f32_gpu(ln, w[L + "attn.c_attn.weight"])
            att = ops.attention_gen2_f32_gpu(qkv, kc, vc, pos, w[L + "attn.c_attn.bias"], heads=HEADS)
            h, ln = proj_ln(att, L + "attn.c_proj.", h, L + "ln_2.", self.sk[0])
            f = ops.gemm_auto_bias_gelu_f32_gpu(ln, w[L + "mlp.c_fc.weight"], w[L + "mlp.c_fc.bias"])
            h, ln = proj_ln(f, L + "mlp.c_proj.", h, nxt, self.sk[1])
        logits = ops.gemm_nt_f32_gpu_mps(ops.view(ln, [1, D], offset=(T - 1) * D), w[P + "wte.weight"])
        return logits, ops.argmax_f32_gpu(logits)

    def _ids(self, ids) -> Tensor:
        if isinstance(ids, Tensor):
            return ids if ids.device == "gpu" else Tensor(ids.t.to(self.positions.device))
        return Tensor(torch.as_tensor(np.asarray(ids, np.int64).reshape(-1)).to(self.positions.device))

    def run(self, ids, pos: int):
        """T = len(ids) new tokens at positions pos..pos+T-1 -> (logits f32[1, 50257] of the last one, its argmax
        i64[1]), both the compiled forward's own buffers (overwritten by the next call). Requires pos + T <= 1024."""
        ids = self._ids(ids)
        T = ids.shape[0]
        if not (T >= 1 and 0 <= pos and pos + T <= N_POS):
            raise ValueError(f"generate: positions {pos}..{pos + T - 1} outside the {N_POS}-row caches")
        p = Tensor(self.positions[pos:pos + 1])
        if T == 1:
            return self.step(ids, p)
        return self.chunk_model.run_inplace(ids, p)

    def __call__(self, ids, pos: int):
        """Reference model(ids, pos) call: logits f32[1, 50257] of the last new token (a host copy)."""
        return self.run(ids, pos)[0].numpy()

    def prefill(self, ids: np.ndarray) -> None:
        """Fills the caches with the prompt in one chunk forward at position 0."""
        self.run(ids, 0)


def generate(model: Gpt2Generator, prompt: list[int], n_new: int) -> list[int]:
    """Greedy generation (reference models/gpt2.py:335-344): one prefill call, then one decode call per new token.
    Each step's argmax stays on the device and feeds the next step directly; the tokens come back in one copy."""
    out = torch.empty(n_new, dtype=torch.int64, device=model.positions.device)
    _, am = model.run(prompt, 0)
    pos = len(prompt)
    for i in range(n_new):
        out[i:i + 1].copy_(am.t)
        if i + 1 == n_new:
            break
        _, am = model.run(Tensor(out[i:i + 1]), pos)
        pos += 1
    return [int(v) for v in out.cpu()]


def build_decode(sd: dict[str, np.ndarray]):
    """The reference's `build_decode(sd, device="gpu")` (models/gpt2.py:161-249) through lk.compile: one decode step
    whose per-layer K / V caches are `lk.persistent_buffer`s (model state that persists across calls; the step
    writes row `pos` in place and attends over rows 0..pos). Inputs tok i64[1], pos i64[1] (device tensors) ->
    logits f32[1, 50257]. The reference's op sequence (gemv4, attention_decode_split, add_bias_layernorm2, the tied
    LM head); its CPU embedding lookups are one device kernel here. Returns the lk.CompiledModel."""
    import lokinfer_amd as lk

    w = {k: from_numpy(v, device="gpu", copy=True) for k, v in sd.items()}
    P = "transformer."

    def fn(tok, pos):
        caches = [(lk.persistent_buffer(lk.f32, [N_POS, D]), lk.persistent_buffer(lk.f32, [N_POS, D]))
                  for _ in range(N_LAYER)]
        h = ops.embedding2_add_f32_gpu(w[P + "wte.weight"], tok, w[P + "wpe.weight"], pos)
        ln = ops.layernorm_f32_gpu(h, w[P + "h.0.ln_1.weight"], w[P + "h.0.ln_1.bias"], eps=LN_EPS)
        for i, (kc, vc) in enumerate(caches):
            L = f"{P}h.{i}."
            nxt = f"{P}h.{i + 1}.ln_1." if i + 1 < N_LAYER else P + "ln_f."
            qkv = ops.gemv4_f32_gpu(ln, w[L + "attn.c_attn.weight"])
            att = ops.attention_decode_split_f32_gpu(qkv, kc, vc, pos, w[L + "attn.c_attn.bias"], heads=HEADS)
            o = ops.gemv4_f32_gpu(att, w[L + "attn.c_proj.weight"])
            h, ln = ops.add_bias_layernorm2_f32_gpu(o, w[L + "attn.c_proj.bias"], h, w[L + "ln_2.weight"],
                                                    w[L + "ln_2.bias"], eps=LN_EPS)
            f = ops.gemv4_f32_gpu(ln, w[L + "mlp.c_fc.weight"], w[L + "mlp.c_fc.bias"], act="gelu")
            o = ops.gemv4_f32_gpu(f, w[L + "mlp.c_proj.weight"])
            h, ln = ops.add_bias_layernorm2_f32_gpu(o, w[L + "mlp.c_proj.bias"], h, w[nxt + "weight"], w[nxt + "bias"],
                                                    eps=LN_EPS)
        return ops.gemm_nt_f32_gpu_mps(ln, w[P + "wte.weight"])

    return lk.compile(fn, input_types=[lk.TensorType(lk.i64, [1]), lk.TensorType(lk.i64, [1])])
