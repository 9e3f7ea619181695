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


# ---- chunked generate (reference build_generate / generate, models/gpt2.py:250-344; its tests compare against
# HF's full forward and HF generate, tests/models/test_gpt2.py:64-106) -------------------------------------------

GEN_PROMPT = [464, 3290, 286, 4881, 318, 6342, 13, 383, 3139, 286]  # tests/models/test_gpt2.py:69


@torch.no_grad()
def last_logits(m, ids) -> np.ndarray:
    """Logits of the last token of the full causal forward over ids -> f32[1, V]."""
    return m(torch.as_tensor(np.asarray(ids, np.int64))[None]).logits[0, -1:].numpy()


@torch.no_grad()
def greedy(m, prompt, n_new: int) -> list[int]:
    """HF generate(do_sample=False) continuation tokens."""
    out = m.generate(torch.tensor([list(prompt)]), max_new_tokens=n_new, do_sample=False, pad_token_id=50256,
                     attention_mask=torch.ones(1, len(prompt), dtype=torch.int64))
    return out[0, len(prompt):].tolist()
