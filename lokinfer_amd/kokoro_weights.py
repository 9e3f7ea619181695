"""Kokoro-82M-shaped parameters and synthetic inputs (the 59- and 487-token benchmark forwards).

Parameter names and shapes follow the Kokoro-82M (StyleTTS2 + iSTFTNet) state dict as the reference's graph
builder reads it (models/kokoro/model.py in lariaus/lokinfer; module shapes bench/research/kokoro/
shapes_510.json), with weight norm already folded (`.weight` instead of `.weight_g` / `.weight_v`, as the
reference's fold_weights produces, model.py:30-47).

Random init (seeded): every weight ~ N(0, 1) / sqrt(fan_in) (fan_in = in_features or Ci * K); biases
~ N(0, 1) / sqrt(fan_in); LayerNorm weights 1 + 0.1 N(0, 1), biases 0.1 N(0, 1); Snake alphas exp(0.1 N(0, 1));
embeddings N(0, 1). One documented exception: the F0 projection bias is 150 (Hz), so the predicted F0 sits in
the voiced range of real speech and the harmonic (sine) branch of the source is exercised rather than only its
noise branch; and conv_post's weight is scaled by 0.1 so the log-magnitudes the iSTFT exponentiates stay O(1).
"""
from __future__ import annotations

import numpy as np

STYLE = 128
HID = 512
N_TOKENS = 178


def _resblk(p: str, cin: int, cout: int, upsample: bool) -> dict:
    s = {p + ".conv1.weight": (cout, cin, 3), p + ".conv1.bias": (cout,),
         p + ".conv2.weight": (cout, cout, 3), p + ".conv2.bias": (cout,),
         p + ".norm1.fc.weight": (2 * cin, STYLE), p + ".norm1.fc.bias": (2 * cin,),
         p + ".norm2.fc.weight": (2 * cout, STYLE), p + ".norm2.fc.bias": (2 * cout,)}
    if cin != cout:
        s[p + ".conv1x1.weight"] = (cout, cin, 1)
    if upsample:
        s[p + ".pool.weight"] = (cin, 1, 3)
        s[p + ".pool.bias"] = (cin,)
    return s


def _resblock1(p: str, ch: int, k: int) -> dict:
    s = {}
    for j in range(3):
        s[f"{p}.convs1.{j}.weight"] = (ch, ch, k)
        s[f"{p}.convs1.{j}.bias"] = (ch,)
        s[f"{p}.convs2.{j}.weight"] = (ch, ch, k)
        s[f"{p}.convs2.{j}.bias"] = (ch,)
        s[f"{p}.adain1.{j}.fc.weight"] = (2 * ch, STYLE)
        s[f"{p}.adain1.{j}.fc.bias"] = (2 * ch,)
        s[f"{p}.adain2.{j}.fc.weight"] = (2 * ch, STYLE)
        s[f"{p}.adain2.{j}.fc.bias"] = (2 * ch,)
        s[f"{p}.alpha1.{j}"] = (1, ch, 1)
        s[f"{p}.alpha2.{j}"] = (1, ch, 1)
    return s


def _lstm(p: str, i: int, h: int) -> dict:
    s = {}
    for sfx in ("", "_reverse"):
        s[f"{p}.weight_ih_l0{sfx}"] = (4 * h, i)
        s[f"{p}.weight_hh_l0{sfx}"] = (4 * h, h)
        s[f"{p}.bias_ih_l0{sfx}"] = (4 * h,)
        s[f"{p}.bias_hh_l0{sfx}"] = (4 * h,)
    return s


def param_shapes() -> dict[str, tuple]:
    s: dict[str, tuple] = {}
    E = "bert.embeddings."
    s.update({E + "word_embeddings.weight": (N_TOKENS, 128), E + "position_embeddings.weight": (512, 128),
              E + "token_type_embeddings.weight": (2, 128), E + "LayerNorm.weight": (128,),
              E + "LayerNorm.bias": (128,),
              "bert.encoder.embedding_hidden_mapping_in.weight": (768, 128),
              "bert.encoder.embedding_hidden_mapping_in.bias": (768,)})
    L = "bert.encoder.albert_layer_groups.0.albert_layers.0."
    for n in ("query", "key", "value", "dense"):
        s[L + f"attention.{n}.weight"] = (768, 768)
        s[L + f"attention.{n}.bias"] = (768,)
    s.update({L + "attention.LayerNorm.weight": (768,), L + "attention.LayerNorm.bias": (768,),
              L + "ffn.weight": (2048, 768), L + "ffn.bias": (2048,), L + "ffn_output.weight": (768, 2048),
              L + "ffn_output.bias": (768,), L + "full_layer_layer_norm.weight": (768,),
              L + "full_layer_layer_norm.bias": (768,),
              "bert_encoder.weight": (HID, 768), "bert_encoder.bias": (HID,)})
    # prosody predictor
    for i in range(3):
        s.update(_lstm(f"predictor.text_encoder.lstms.{2 * i}", HID + STYLE, HID // 2))
        s[f"predictor.text_encoder.lstms.{2 * i + 1}.fc.weight"] = (2 * HID, STYLE)
        s[f"predictor.text_encoder.lstms.{2 * i + 1}.fc.bias"] = (2 * HID,)
    s.update(_lstm("predictor.lstm", HID + STYLE, HID // 2))
    s.update({"predictor.duration_proj.linear_layer.weight": (50, HID),
              "predictor.duration_proj.linear_layer.bias": (50,)})
    s.update(_lstm("predictor.shared", HID + STYLE, HID // 2))
    for name in ("F0", "N"):
        s.update(_resblk(f"predictor.{name}.0", HID, HID, False))
        s.update(_resblk(f"predictor.{name}.1", HID, HID // 2, True))
        s.update(_resblk(f"predictor.{name}.2", HID // 2, HID // 2, False))
        s[f"predictor.{name}_proj.weight"] = (1, HID // 2, 1)
        s[f"predictor.{name}_proj.bias"] = (1,)
    # text encoder
    s["text_encoder.embedding.weight"] = (N_TOKENS, HID)
    for i in range(3):
        s[f"text_encoder.cnn.{i}.0.weight"] = (HID, HID, 5)
        s[f"text_encoder.cnn.{i}.0.bias"] = (HID,)
        s[f"text_encoder.cnn.{i}.1.gamma"] = (HID,)
        s[f"text_encoder.cnn.{i}.1.beta"] = (HID,)
    s.update(_lstm("text_encoder.lstm", HID, HID // 2))
    # decoder
    s.update({"decoder.F0_conv.weight": (1, 1, 3), "decoder.F0_conv.bias": (1,),
              "decoder.N_conv.weight": (1, 1, 3), "decoder.N_conv.bias": (1,),
              "decoder.asr_res.0.weight": (64, HID, 1), "decoder.asr_res.0.bias": (64,)})
    s.update(_resblk("decoder.encode", HID + 2, 1024, False))
    for i in range(4):
        s.update(_resblk(f"decoder.decode.{i}", 1024 + 64 + 2, 1024 if i < 3 else HID, i == 3))
    G = "decoder.generator."
    s.update({G + "m_source.l_linear.weight": (1, 9), G + "m_source.l_linear.bias": (1,),
              G + "noise_convs.0.weight": (256, 22, 12), G + "noise_convs.0.bias": (256,),
              G + "noise_convs.1.weight": (128, 22, 1), G + "noise_convs.1.bias": (128,),
              G + "ups.0.weight": (HID, 256, 20), G + "ups.0.bias": (256,),
              G + "ups.1.weight": (256, 128, 12), G + "ups.1.bias": (128,),
              G + "conv_post.weight": (22, 128, 7), G + "conv_post.bias": (22,)})
    s.update(_resblock1(G + "noise_res.0", 256, 7))
    s.update(_resblock1(G + "noise_res.1", 128, 11))
    for i, ch in enumerate((256, 128)):
        for j, k in enumerate((3, 7, 11)):
            s.update(_resblock1(f"{G}resblocks.{3 * i + j}", ch, k))
    return s


def _fan_in(name: str, shape: tuple) -> int:
    if len(shape) == 3:  # conv [Co, Ci, K] or convT [Ci, Co, K]
        if ".ups." in name or ".pool." in name:
            return shape[0] * shape[2] if ".ups." in name else shape[2]
        return shape[1] * shape[2]
    if len(shape) == 2:
        return shape[1]
    return 1


def random_weights(seed: int = 82) -> dict[str, np.ndarray]:
    sd: dict[str, np.ndarray] = {}
    shapes = param_shapes()
    for i, k in enumerate(sorted(shapes)):
        shape = shapes[k]
        z = np.random.default_rng(seed * 100003 + i).standard_normal(shape)
        if k.endswith(("LayerNorm.weight", "layer_norm.weight", ".gamma")):
            a = 1.0 + 0.1 * z
        elif k.endswith(("LayerNorm.bias", "layer_norm.bias", ".beta")):
            a = 0.1 * z
        elif ".alpha" in k:
            a = np.exp(0.1 * z)
        elif "embeddings" in k or k.endswith("embedding.weight"):
            a = z
        elif k.endswith(".bias") or "bias_ih" in k or "bias_hh" in k:
            fan = shapes[k.replace("bias_ih", "weight_ih").replace("bias_hh", "weight_hh").replace(".bias", ".weight")]
            a = z / np.sqrt(_fan_in(k, fan))
        else:
            a = z / np.sqrt(_fan_in(k, shape))
        sd[k] = a.astype(np.float32)
    sd["predictor.F0_proj.bias"] = np.array([150.0], np.float32)
    # conv_post emits log-magnitudes that the iSTFT exponentiates: x0.1 keeps them O(1) like a trained model's.
    sd["decoder.generator.conv_post.weight"] *= np.float32(0.1)
    return sd


def inputs(tokens: int, seed: int = 59):
    """(ids i64[T], ref_s f32[256], dur i64[T], noise f32[600 F, 9]) for a T-token forward: ids uniform in
    [0, 178) with pad id 0 at both ends (T counts the pads), ref_s ~ N(0, 1), durations uniform 2..8,
    F = sum(dur), SineGen noise ~ N(0, 1)."""
    rng = np.random.default_rng(seed * 7919 + tokens)
    ids = rng.integers(0, N_TOKENS, tokens).astype(np.int64)
    ids[0] = ids[-1] = 0
    ref_s = rng.standard_normal(256).astype(np.float32)
    dur = rng.integers(2, 9, tokens).astype(np.int64)
    f = int(dur.sum())
    noise = rng.standard_normal((600 * f, 9)).astype(np.float32)
    return ids, ref_s, dur, noise
