"""TEST INFRASTRUCTURE ONLY. GPT-2 124M decode oracle: transformers.GPT2LMHeadModel(GPT2Config()) built
locally (no download) and loaded with the same seeded weights as the GPU path; one step with a 512-token
past_key_values (reference models/gpt2.py:161-249 semantics; tests/models/test_gpt2.py:54-61 invariant: the
decode step at pos p equals the full forward's row p).

Also the PyTorch f32 CPU baseline of the bench (the reference's CPU decode uses Accelerate/NEON only,
kernels/cpu/decode.cpp)."""
from __future__ import annotations

import numpy as np
import torch

PROMPT_SEED, NEXT_SEED, PROMPT_LEN, VOCAB = 4242, 4243, 512, 50257


def decode_inputs():
    ids = np.random.default_rng(PROMPT_SEED).integers(0, VOCAB, PROMPT_LEN, dtype=np.int64)
    nxt = int(np.random.default_rng(NEXT_SEED).integers(0, VOCAB))
    return ids, nxt


def model(sd: dict[str, np.ndarray], dtype=torch.float32):
    from transformers import GPT2Config, GPT2LMHeadModel

    cfg = GPT2Config()
    cfg.attn_implementation = "eager"
    m = GPT2LMHeadModel(cfg).eval()
    state = {k: torch.from_numpy(v) for k, v in sd.items()}
    state["lm_head.weight"] = state["transformer.wte.weight"]
    missing, unexpected = m.load_state_dict(state, strict=False)
    assert not unexpected, unexpected
    assert all(k.endswith("attn.bias") or k.endswith("masked_bias") for k in missing), missing
    return m.to(dtype)


@torch.no_grad()
def prefill(m, ids: np.ndarray):
    out = m(torch.from_numpy(ids)[None], use_cache=True)
    return out.past_key_values


@torch.no_grad()
def decode_step(m, past, tok: int):
    out = m(torch.tensor([[tok]]), past_key_values=past, use_cache=True)
    return out.logits[0, -1].numpy(), out.past_key_values
