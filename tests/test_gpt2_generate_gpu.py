"""GPT-2 124M chunked prefill + greedy generation on the GPU vs the transformers oracle, mirroring the reference's
build_generate tests (tests/models/test_gpt2.py:64-106): one prefill call then one call per token must match HF
generate token for token; every chunk's last-row logits (chunks at pos > 0, longer than a 32-query block, not
aligned, interleaved with decode steps) match HF's full forward within max rel err 1e-4."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def setup(gpu):
    from lokinfer_amd import gpt2 as G
    from oracle import gpt2 as O

    sd = G.random_weights()
    return G, O, sd, O.model(sd)


def rel(got, exp):
    return np.abs(got - exp).max() / np.abs(exp).max()


def test_prefill_logits_and_generate(setup):
    G, O, sd, m = setup
    model = G.Gpt2Generator(sd)
    got = model(O.GEN_PROMPT, 0)
    assert rel(got, O.last_logits(m, O.GEN_PROMPT)) <= 1e-4
    hf = O.greedy(m, O.GEN_PROMPT, 32)
    assert G.generate(G.Gpt2Generator(sd), O.GEN_PROMPT, 32) == hf  # fresh caches
    # the reference op sequence for the decode steps (fused=False) generates the same tokens
    assert G.generate(G.Gpt2Generator(sd, fused=False, sk=(0, 0)), O.GEN_PROMPT, 8) == hf[:8]


def test_two_chunk_prefill(setup):
    G, O, sd, m = setup
    model = G.Gpt2Generator(sd)
    p = O.GEN_PROMPT
    model(p[:6], 0)
    assert rel(model(p[6:], 6), O.last_logits(m, p)) <= 1e-4


def test_multi_chunk_prefill(setup):
    G, O, sd, m = setup
    model = G.Gpt2Generator(sd)
    ids = np.random.default_rng(3).integers(0, G.VOCAB, 300).astype(np.int64)
    pos = 0
    for n in (40, 70, 1, 117, 1, 71):
        got = model(ids[pos:pos + n], pos)
        pos += n
        assert rel(got, O.last_logits(m, ids[:pos])) <= 1e-4, (pos, n)


def test_prefill_512_then_decode(setup):
    """The decode benchmark's configuration reached through one 512-token prefill chunk instead of 512 steps: the
    step at pos 512 matches the oracle's decode step and its argmax."""
    G, O, sd, m = setup
    ids, nxt = O.decode_inputs()
    ref, _ = O.decode_step(m, O.prefill(m, ids), nxt)
    model = G.Gpt2Generator(sd)
    model.prefill(ids)
    got = model([nxt], 512)[0]
    assert rel(got, ref) <= 1e-4
    assert int(np.argmax(got)) == int(np.argmax(ref))


def test_chunk_graph_equals_eager(setup):
    G, O, sd, m = setup
    a, b = G.Gpt2Generator(sd), G.Gpt2Generator(sd, chunk_graph=True)
    ids = np.random.default_rng(5).integers(0, G.VOCAB, 96).astype(np.int64)
    for pos in (0, 32, 64):  # the same T three times: graph capture, then replays
        la, lb = a(ids[pos:pos + 32], pos), b(ids[pos:pos + 32], pos)
        assert np.array_equal(la, lb), pos


def test_generate_to_cache_capacity(setup):
    """A 1000-token prompt in one chunk, then decode steps up to position 1023 (the last cache row; 16 decode chunks
    and 32 key tiles of the cache attention): every step's logits match HF's full forward over the tokens so far."""
    G, O, sd, m = setup
    model = G.Gpt2Generator(sd)
    ids = np.random.default_rng(9).integers(0, G.VOCAB, 1024).astype(np.int64)
    got = model(ids[:1000], 0)
    assert rel(got, O.last_logits(m, ids[:1000])) <= 1e-4
    for pos in (1000, 1001, 1023):
        if pos > 1001:
            for p in range(1002, pos):
                model(ids[p:p + 1], p)
        got = model(ids[pos:pos + 1], pos)
        assert rel(got, O.last_logits(m, ids[:pos + 1])) <= 1e-4, pos
    with pytest.raises(ValueError):
        model(ids[:2], 1023)  # past the cache: refused on the host


def test_capture_with_collectable_models(setup):
    """Regression: models hold their compiled function and it holds them back, so only the cycle collector frees
    them, and a collection during a graph capture destroyed their captured graphs mid-capture. Unreachable models
    are left behind and the collector is made to run on (nearly) every allocation while a new model captures; the
    capture must succeed and give the eager logits."""
    import gc

    G, O, sd, m = setup
    for _ in range(2):
        d = G.Gpt2Generator(sd)
        d([5, 6, 7], 0)
        d([8], 3)  # captures the decode graph
        del d  # now only reachable through its own cycle
    old = gc.get_threshold()
    gc.set_threshold(1)
    try:
        a = G.Gpt2Generator(sd, graph=True)
        a([5, 6, 7], 0)
        la = a([8], 3)
    finally:
        gc.set_threshold(*old)
    assert gc.isenabled()
    b = G.Gpt2Generator(sd, graph=False)
    b([5, 6, 7], 0)
    assert np.array_equal(la, b([8], 3))
