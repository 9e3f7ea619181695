"""Pins the GPT-2 oracle (transformers GPT2LMHeadModel built locally with the seeded weights): the decode step
at position p equals row p of the full causal forward (reference tests/models/test_gpt2.py:54-61), and the
model's first block matches this repo's numpy restatement of the layer (oracle/kernels.py)."""
import numpy as np
import torch

from lokinfer_amd import gpt2 as G
from oracle import gpt2 as O
from oracle import kernels as K


def test_weights_are_seeded_and_shaped():
    sd = G.random_weights()
    assert sd["transformer.h.3.mlp.c_fc.weight"].shape == (768, 3072)
    assert abs(float(sd["transformer.wte.weight"].std()) - 0.02) < 1e-3
    assert abs(float(sd["transformer.ln_f.weight"].mean()) - 1.0) < 1e-2
    assert np.array_equal(G.random_weights()["transformer.wpe.weight"], sd["transformer.wpe.weight"])


def test_decode_step_equals_full_forward_row():
    sd = G.random_weights()
    m = O.model(sd, torch.float64)
    ids = np.random.default_rng(1).integers(0, 50257, 17)
    with torch.no_grad():
        full = m(torch.from_numpy(ids)[None]).logits[0].numpy()
    past = O.prefill(m, ids[:16])
    step, _ = O.decode_step(m, past, int(ids[16]))
    np.testing.assert_allclose(step, full[16], rtol=1e-9, atol=1e-9)


def test_first_block_matches_numpy_restatement():
    sd = G.random_weights()
    m = O.model(sd, torch.float64)
    ids = np.array([5, 17, 900])
    L = "transformer.h.0."
    h = sd["transformer.wte.weight"][ids].astype(np.float64) + sd["transformer.wpe.weight"][:3]
    a = K.layernorm(h, sd[L + "ln_1.weight"], sd[L + "ln_1.bias"], 1e-5)
    qkv = K.gemm(a, sd[L + "attn.c_attn.weight"])
    att = K.attention_qkv(qkv, sd[L + "attn.c_attn.bias"], 12, causal=True)
    h = h + K.gemm(att, sd[L + "attn.c_proj.weight"], sd[L + "attn.c_proj.bias"])
    f = K.gemm(K.layernorm(h, sd[L + "ln_2.weight"], sd[L + "ln_2.bias"], 1e-5), sd[L + "mlp.c_fc.weight"],
               sd[L + "mlp.c_fc.bias"], act="gelu")
    h = h + K.gemm(f, sd[L + "mlp.c_proj.weight"], sd[L + "mlp.c_proj.bias"])
    with torch.no_grad():
        hs = m.transformer(torch.from_numpy(ids)[None], output_hidden_states=True).hidden_states[1][0].numpy()
    np.testing.assert_allclose(h, hs, rtol=1e-9, atol=1e-9)


def test_greedy_equals_argmax_of_full_forward():
    """HF generate's greedy continuation is, token by token, the argmax of the full forward over the tokens so far
    (pins the generate oracle against the forward oracle pinned above)."""
    sd = G.random_weights()
    m = O.model(sd)
    toks = O.greedy(m, O.GEN_PROMPT, 6)
    seq = list(O.GEN_PROMPT)
    for t in toks:
        assert int(np.argmax(O.last_logits(m, seq)[0])) == t
        seq.append(t)
