"""The runtime's IR library through its C-ABI (include/lokinfer_rt.h), against golden outputs written by the
reference's own IR library (tests/golden/make_ir_golden.py over oracle/_ref/lkm-ref-tool, built from lariaus/lokinfer
src/ir + src/compiler): the printed model, each pass stage, the .lkm v2 bytes and the .lkm read back must be
byte-identical. No GPU needed."""
import re
from pathlib import Path

import numpy as np
import pytest

from lokinfer_amd._lib import LokinferError
from lokinfer_amd.rt import Model, dim_canonical

GOLD = Path(__file__).resolve().parent / "golden" / "ir"
CASES = sorted(p.stem for p in GOLD.glob("*.lkir"))
SIZES = {"f32": 4, "f16": 2, "bf16": 2, "i8": 1, "u8": 1, "i16": 2, "i32": 4, "i64": 8, "bool": 1}


def fixture_bytes(name: str, n: int) -> bytes:
    """Byte k of constant `name`: (k * 29 + sum of the name's bytes) mod 251 (oracle/lkm_ref_tool.cpp)."""
    s = sum(name.encode())
    return ((np.arange(n, dtype=np.int64) * 29 + s) % 251).astype(np.uint8).tobytes()


def internal_constants(text: str):
    for name, dt, shape in re.findall(r'const\.internal @"([^"]+)"[^:]*: tensor<(\w+)\[([^\]]*)\]>', text):
        n = SIZES[dt]
        for d in (x for x in shape.split(",") if x.strip()):
            n *= int(d)
        yield name, n


def test_corpus_present():
    assert len(CASES) >= 5


@pytest.mark.parametrize("case", CASES)
def test_print_matches_reference(case):
    m = Model.parse((GOLD / f"{case}.lkir").read_text())
    assert m.text() == (GOLD / f"{case}.print.txt").read_text()
    # and printing is a fixed point of parsing
    assert Model.parse(m.text()).text() == m.text()


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("stage,passes", [("bufferize", "dce,bufferize"), ("plan", "dce,bufferize,plan-memory"),
                                          ("pipeline", "pipeline")])
def test_passes_match_reference(case, stage, passes):
    m = Model.parse((GOLD / f"{case}.lkir").read_text())
    m.run_passes(passes)
    assert m.text() == (GOLD / f"{case}.{stage}.txt").read_text()


@pytest.mark.parametrize("case", [c for c in CASES if (GOLD / f"{c}.lkm").exists()])
def test_lkm_bytes_match_reference(case, tmp_path):
    src = (GOLD / f"{case}.lkir").read_text()
    m = Model.parse(src)
    m.run_passes("pipeline")
    for name, n in internal_constants(src):
        m.set_constant(name, fixture_bytes(name, n))
    gold = (GOLD / f"{case}.lkm").read_bytes()
    assert m.to_bytes() == gold
    m.save(tmp_path / "x.lkm")
    assert (tmp_path / "x.lkm").read_bytes() == gold
    back = Model.load(GOLD / f"{case}.lkm")
    assert back.text() == (GOLD / f"{case}.lkm.txt").read_text()
    assert back.to_bytes() == gold  # read -> write is the identity
    assert Model.from_bytes(gold).to_bytes() == gold


def test_lkm_rejects_corrupt_files():
    gold = (GOLD / "decode_persistent.lkm").read_bytes()
    for bad, msg in [(b"XKM\0" + gold[4:], "bad magic"), (gold[:40], "too small|truncated"),
                     (gold[:4] + bytes([9, 0, 0, 0]) + gold[8:], "unsupported version"),
                     (gold[:64] + bytes(len(gold) - 64), "corrupt|bad|verify")]:
        with pytest.raises(LokinferError, match=msg):
            Model.from_bytes(bad)


def test_external_constants_cannot_be_saved_until_internalized():
    m = Model.parse((GOLD / "mutable_chain.lkir").read_text())
    with pytest.raises(LokinferError, match="internalized"):
        m.to_bytes()
    w = np.arange(128 * 128, dtype=np.float32).reshape(128, 128)
    m.internalize({"ext0": w})
    b = m.to_bytes()
    assert "const.internal @\"ext0\"" in Model.from_bytes(b).text()


@pytest.mark.parametrize("text,canon", [
    ("2*(N + 1)", "2*N + 2"), ("(2*F - 1) // 2 + 1", "F"), ("N + M + M - 2*M + 7", "N + 7"),
    ("M*N*2", "2*M*N"), ("max(N, M)", "max(M, N)"), ("ceildiv(120*F + 1, 5)", "24*F + 1"),
    ("(N + 3) % 4", "(N + 3) % 4"), ("-N + 3*N", "2*N"), ("600*F // 600", "F"), ("7 - 3", "4")])
def test_dim_canonical_forms(text, canon):
    assert dim_canonical(text) == canon


@pytest.mark.parametrize("body,msg", [
    # an in-place write to an immutable input
    ("exec(%x: buffer<f32[4]>) {\n kernel \"k_f32_gpu\"(%x) {inout = [0]}\n return\n }", "mutable input"),
    # returning a mutable input
    ("exec(%x: buffer<f32[4]> mutable) {\n return %x\n }", "mutable input"),
    # a host read of a GPU-resident value
    ("exec(%x: tensor<f32[4]>) {\n %d = kernel \"n_i64_gpu\"(%x) : tensor<i64[1]>\n dim.read %d[0] -> F\n"
     " %y = kernel \"e_f32_gpu\"(%x) : tensor<f32[F]>\n return %y\n }", "dim.read"),
    # a symbol nothing binds
    ("exec(%x: tensor<f32[4]>) {\n %y = kernel \"e_f32_gpu\"(%x) : tensor<f32[Q]>\n return %y\n }", "unbound symbol"),
    # a GPU kernel reading a value resident on the CPU
    ("exec(%x: tensor<f32[4]>) {\n %a = kernel \"h_f32_cpu\"(%x) : tensor<f32[4]>\n"
     " %b = kernel \"g_f32_gpu\"(%a) : tensor<f32[4]>\n return %b\n }", "resident on cpu"),
])
def test_verifier_rejects(body, msg):
    with pytest.raises(LokinferError, match=msg):
        Model.parse("model {\n init {\n return\n }\n " + body + "\n}\n")


def test_parse_errors_name_the_line():
    with pytest.raises(LokinferError, match="line 3"):
        Model.parse("model {\n  init {\n    bogus\n  }\n}\n")


# ---- the reference's lit-test models (tests/golden/ir/lit, written by tests/golden/make_ir_lit_golden.py) ----------

LIT = GOLD / "lit"
LIT_CASES = sorted(p.stem for p in LIT.glob("*.lkir"))


def test_lit_corpus_present():
    assert len(LIT_CASES) >= 25


@pytest.mark.parametrize("case", LIT_CASES)
def test_lit_stage_matches_reference(case):
    """The passes the reference's lit test runs (or none) give the reference library's text, or both reject."""
    src = (LIT / f"{case}.lkir").read_text()
    passes = (LIT / f"{case}.stage").read_text().strip()
    want = (LIT / f"{case}.stage.txt").read_text()

    def go():
        m = Model.parse(src)
        if passes != "-":
            m.run_passes(passes)
        return m.text()

    if want == "rejected\n":
        with pytest.raises(LokinferError):
            go()
    else:
        assert go() == want


@pytest.mark.parametrize("case", [c for c in LIT_CASES if (LIT / f"{c}.pipeline.txt").exists()])
def test_lit_pipeline_and_lkm_match_reference(case, tmp_path):
    src = (LIT / f"{case}.lkir").read_text()
    m = Model.parse(src)
    m.run_passes("pipeline")
    assert m.text() == (LIT / f"{case}.pipeline.txt").read_text()
    lkm = LIT / f"{case}.lkm"
    if not lkm.exists():
        return
    for name, n in internal_constants(src):
        m.set_constant(name, fixture_bytes(name, n))
    gold = lkm.read_bytes()
    assert m.to_bytes() == gold
    back = Model.from_bytes(gold)
    assert back.text() == (LIT / f"{case}.lkm.txt").read_text()
    assert back.to_bytes() == gold


@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_const_inline_half_rounding(dt):
    """const.inline f16 / bf16 data rounds to nearest even like numpy's float16 / torch's bfloat16 casts, including
    subnormals, exact ties, overflow to infinity and the largest finite values; printing gives the rounded value."""
    import torch

    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(400) * 10.0 ** rng.integers(-9, 6, 400),
                        [0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -25,
                         1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, 3.0e38, 1 + 2.0 ** -8, 1 + 3 * 2.0 ** -8]]).astype(np.float32)
    text = ("model {\n init {\n return\n }\n exec() {\n %c = const.inline dense<["
            + ", ".join(repr(float(v)) for v in x) + f"]> : tensor<{dt}[{len(x)}]>\n return %c\n }}\n}}\n")
    printed = Model.parse(text).text()
    # the text has 9 significant digits: enough to name a float32 (so every f16 / bf16 value) exactly
    got = np.array([float(v) for v in re.search(r"dense<\[(.*?)\]>", printed).group(1).split(", ")], np.float32)
    with np.errstate(over="ignore"):
        if dt == "f16":
            assert np.array_equal(got.astype(np.float16).view(np.uint16), x.astype(np.float16).view(np.uint16))
        else:
            b = lambda a: torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy()  # noqa: E731
            assert np.array_equal(b(got), b(x))
