"""Pins the Qwen3 LM oracle (oracle/qwen3.py): with rounding off, its basic graph equals transformers'
Qwen3ForCausalLM (float64, built locally, same weights) for a whole prompt and for the same prompt fed in chunks
and single decode steps over the cache (reference tests/models/test_qwen3_asr.py checks chunked prefill + decode
against its golden data the same way); RoPE, RMSNorm and GQA attention against closed forms and torch; the f16
rounding points of the contract on small cases."""
import numpy as np
import pytest
import torch

from lokinfer_amd.qwen3 import Qwen3Config, random_weights
from oracle import qwen3 as Q

CFG = Qwen3Config(layers=2, d=256, qh=4, kvh=2, ffn=512)  # the real vocabulary: the pad id is a token
rng = np.random.default_rng(11)


@pytest.fixture(scope="module")
def tiny():
    sd = random_weights(CFG, 5)
    return sd, Q.hf_model(sd, CFG)


def _hf_last(m, sd, ids, audio):
    o = Q.Ops(np.float64, rounding=False)
    emb = o.scatter_audio(o.embedding(ids, sd["embed"]), ids, audio)
    with torch.no_grad():
        return m(inputs_embeds=torch.from_numpy(emb)[None]).logits[0, -1:].numpy()


def test_basic_graph_equals_hf_float64(tiny):
    sd, m = tiny
    ids = rng.integers(0, 150000, 20)
    ids[3:9] = Q.PAD_ID  # six audio rows scattered into the embeddings
    audio = rng.standard_normal((6, CFG.d)) * 0.5
    ref = _hf_last(m, sd, ids, audio)
    got = Q.OracleLm(sd, CFG, Q.Ops(np.float64, rounding=False), 32)(ids, audio, 0)
    assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max()


def test_chunks_and_decode_steps_equal_full_forward(tiny):
    sd, m = tiny
    ids = rng.integers(0, 150000, 16)
    ids[2:6] = Q.PAD_ID
    audio = rng.standard_normal((4, CFG.d)) * 0.5
    lm = Q.OracleLm(sd, CFG, Q.Ops(np.float64, rounding=False), 24)
    pos = 0
    for n in (5, 7, 1, 1, 2):
        k0, k1 = np.count_nonzero(ids[:pos] == Q.PAD_ID), np.count_nonzero(ids[:pos + n] == Q.PAD_ID)
        got = lm(ids[pos:pos + n], audio[k0:k1] if k1 > k0 else np.zeros((1, CFG.d)), pos)
        pos += n
        ref = _hf_last(m, sd, ids[:pos], audio[:k1])
        assert np.abs(got - ref).max() <= 1e-6 * np.abs(ref).max(), pos


def test_rope_closed_forms():
    o = Q.Ops(np.float64, rounding=False)
    x = rng.standard_normal((5, 256))
    np.testing.assert_allclose(o.rope(x[:1], 0), x[:1], rtol=0, atol=0)  # angle 0 at position 0
    y = o.rope(x, 37)
    for h0 in (0, 128):  # each (j, j + 64) pair is rotated: its norm is kept
        n0 = x[:, h0:h0 + 64] ** 2 + x[:, h0 + 64:h0 + 128] ** 2
        n1 = y[:, h0:h0 + 64] ** 2 + y[:, h0 + 64:h0 + 128] ** 2
        np.testing.assert_allclose(n1, n0, rtol=1e-6)
    # pair j = 0 turns by exactly the position (inv_freq[0] = 1)
    a = 37 + 2
    np.testing.assert_allclose(y[2, 0], x[2, 0] * np.cos(a) - x[2, 64] * np.sin(a), rtol=1e-6)


def test_attention_gqa_equals_sdpa():
    o = Q.Ops(np.float64, rounding=False)
    t, pos, qh, kvh = 6, 9, 4, 2
    q = rng.standard_normal((t, 128 * qh))
    kc, vc = rng.standard_normal((20, 128 * kvh)), rng.standard_normal((20, 128 * kvh))
    got = o.attention_gqa(q, kc, vc, pos, qh, kvh)
    Qt = torch.from_numpy(q).view(t, qh, 128).transpose(0, 1)
    K = torch.from_numpy(kc[:pos + t]).view(pos + t, kvh, 128).transpose(0, 1).repeat_interleave(qh // kvh, 0)
    V = torch.from_numpy(vc[:pos + t]).view(pos + t, kvh, 128).transpose(0, 1).repeat_interleave(qh // kvh, 0)
    mask = torch.arange(pos + t)[None, :] <= (pos + torch.arange(t))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(Qt, K, V, attn_mask=mask).transpose(0, 1).reshape(t, -1)
    np.testing.assert_allclose(got, ref.numpy(), rtol=1e-10, atol=1e-12)
    with pytest.raises(ValueError):
        o.attention_gqa(q, kc, vc, 15, qh, kvh)


def test_rounding_points():
    o = Q.Ops(np.float64)
    # rmsnorm of a constant row: h = f16(c / sqrt(c^2 + eps)) rounds to 1 for c = 3, then y = f16(g * 1) = g
    g = np.array([1.5, -0.25] * 4, np.float16)
    np.testing.assert_array_equal(o.rmsnorm(np.full((1, 8), 3.0), g), g[None].astype(np.float64))
    # gemm rounds once: 2049 = 2048 + 1 is not an f16 (spacing 2 above 2048) and rounds to even 2048
    x, w = np.ones((1, 8)), np.full((8, 1), 256.0)
    assert o.gemm(x, w)[0, 0] == 2048.0 and o.gemm(x, w * 1.0 + np.eye(8, 1) / 1.0)[0, 0] == 2048.0
    assert o.add(np.array([[2048.0]]), np.array([[3.0]]))[0, 0] == 2052.0  # 2051 -> 2052 (ties to even)
    with pytest.raises(ValueError):
        o.scatter_audio(np.zeros((3, 8)), np.array([Q.PAD_ID] * 3), np.zeros((2, 8)))
