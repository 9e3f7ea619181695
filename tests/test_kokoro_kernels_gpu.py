"""GPU parity of the Kokoro front-end / signal kernels (the host kernels of the reference's GPU graph, run on the
device here) against the oracle: torch nn.LSTM / F.layer_norm / torch.stft in float64 and the f32 restatement
of the harmonic source (oracle/kokoro.py, reference kernels/cpu/kokoro_signal.cpp:89-192)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kokoro as OK

pytestmark = pytest.mark.gpu

rng = np.random.default_rng(99)


def G(lk, a, dt=np.float32):
    return lk.from_numpy(np.ascontiguousarray(a, dt), device="gpu", copy=True)


def close(got, ref, tol):
    got = got.numpy() if hasattr(got, "numpy") else np.asarray(got)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    err = np.abs(got.astype(np.float64) - ref).max()
    scale = max(1.0, np.abs(ref).max())
    assert err <= tol * scale, f"max err {err:.3e} > {tol:.1e} * {scale:.3e}"


@pytest.mark.parametrize("t,i", [(1, 640), (59, 640), (300, 512), (2435, 640)])
def test_lstm_bidir(gpu, t, i):
    lk = gpu
    h = 256
    x = rng.standard_normal((t, i)).astype(np.float32)
    sd = {}
    for sfx in ("", "_reverse"):
        sd[f"l.weight_ih_l0{sfx}"] = (rng.standard_normal((4 * h, i)) / np.sqrt(i)).astype(np.float32)
        sd[f"l.weight_hh_l0{sfx}"] = (rng.standard_normal((4 * h, h)) / np.sqrt(h)).astype(np.float32)
        sd[f"l.bias_ih_l0{sfx}"] = (rng.standard_normal(4 * h) * 0.1).astype(np.float32)
        sd[f"l.bias_hh_l0{sfx}"] = (rng.standard_normal(4 * h) * 0.1).astype(np.float32)
    ref = OK.Oracle(sd, torch.float64).lstm(torch.from_numpy(x).double(), "l").numpy()
    w_ih = np.concatenate([sd["l.weight_ih_l0"], sd["l.weight_ih_l0_reverse"]])
    w_hh_t = np.concatenate([sd["l.weight_hh_l0"], sd["l.weight_hh_l0_reverse"]]).T
    b = np.concatenate([sd["l.bias_ih_l0"] + sd["l.bias_hh_l0"], sd["l.bias_ih_l0_reverse"] + sd["l.bias_hh_l0_reverse"]])
    got = lk.ops.lstm_bidir_t_f32_gpu(G(lk, x), G(lk, w_ih), G(lk, w_hh_t), G(lk, b))
    close(got, ref, 1e-4)


@pytest.mark.parametrize("t", [1, 59, 487])
def test_lstm2_bidir_equals_two_lstms(gpu, t):
    """lstm2_bidir_t (two BiLSTMs of one length in one recurrence launch, the Kokoro text encoder beside the
    duration encoder) gives each LSTM the bits of its own lstm_bidir_t launch; different input widths."""
    lk = gpu
    h = 256
    sets = []
    for i in (640, 512):
        w_ih = (rng.standard_normal((8 * h, i)) / np.sqrt(i)).astype(np.float32)
        w_hh_t = (rng.standard_normal((h, 8 * h)) / np.sqrt(h)).astype(np.float32)
        b = (rng.standard_normal(8 * h) * 0.1).astype(np.float32)
        x = rng.standard_normal((t, i)).astype(np.float32)
        sets.append(tuple(G(lk, a) for a in (x, w_ih, w_hh_t, b)))
    y1, y2 = lk.ops.lstm2_bidir_t_f32_gpu(*sets[0], *sets[1])
    assert np.array_equal(y1.numpy(), lk.ops.lstm_bidir_t_f32_gpu(*sets[0]).numpy())
    assert np.array_equal(y2.numpy(), lk.ops.lstm_bidir_t_f32_gpu(*sets[1]).numpy())


@pytest.mark.parametrize("t", [1, 59, 2444])
def test_lstm_exchange_paths_agree(gpu, t, monkeypatch):
    """The XCD-local exchange (each direction's workgroups on one XCD, words through its L2) and the agent-scope
    one (LK_LSTM_EXCHANGE=agent) run the same arithmetic: identical bits, for one LSTM and for two in one launch."""
    lk = gpu
    h, i = 256, 640
    w_ih = (rng.standard_normal((8 * h, i)) / np.sqrt(i)).astype(np.float32)
    w_hh_t = (rng.standard_normal((h, 8 * h)) / np.sqrt(h)).astype(np.float32)
    b = (rng.standard_normal(8 * h) * 0.1).astype(np.float32)
    x = rng.standard_normal((t, i)).astype(np.float32)
    a = tuple(G(lk, v) for v in (x, w_ih, w_hh_t, b))
    local = lk.ops.lstm_bidir_t_f32_gpu(*a).numpy()
    local2 = [y.numpy() for y in lk.ops.lstm2_bidir_t_f32_gpu(*a, *a)]
    monkeypatch.setenv("LK_LSTM_EXCHANGE", "agent")
    agent = lk.ops.lstm_bidir_t_f32_gpu(*a).numpy()
    assert np.isfinite(agent).all()
    assert np.array_equal(local, agent)
    assert all(np.array_equal(y, agent) for y in local2)


def test_lstm_bidir_repeated_launches(gpu):
    """Back-to-back launches with alternating lengths, the second one concurrent with work on another stream:
    every result is finite and identical to the first (the cross-workgroup exchange words are reused by every
    launch and by every step of one launch)."""
    lk = gpu
    h, i = 256, 512
    w_ih = (rng.standard_normal((8 * h, i)) / np.sqrt(i)).astype(np.float32)
    w_hh_t = (rng.standard_normal((h, 8 * h)) / np.sqrt(h)).astype(np.float32)
    b = (rng.standard_normal(8 * h) * 0.1).astype(np.float32)
    xs = {t: rng.standard_normal((t, i)).astype(np.float32) for t in (2, 59, 300)}
    args = {t: (G(lk, x), G(lk, w_ih), G(lk, w_hh_t), G(lk, b)) for t, x in xs.items()}
    first = {t: lk.ops.lstm_bidir_t_f32_gpu(*a).numpy() for t, a in args.items()}
    for t, r in first.items():
        assert np.isfinite(r).all(), t
    side = torch.cuda.Stream()
    big = torch.randn(2048, 2048, device="cuda")
    for n in range(60):
        t = (2, 59, 300)[n % 3]
        if n % 2:
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for _ in range(4):
                    big = big @ big * 1e-3
        got = lk.ops.lstm_bidir_t_f32_gpu(*args[t]).numpy()
        assert np.array_equal(got, first[t]), f"launch {n} (T={t}) differs"
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()


def test_repeat_interleave_adaln_concat(gpu):
    lk = gpu
    t, c = 59, 640
    x = rng.standard_normal((t, c)).astype(np.float32)
    dur = rng.integers(0, 9, t).astype(np.int64)
    frames = int(dur.sum())
    got = lk.ops.repeat_interleave_f32_gpu(G(lk, x), G(lk, dur, np.int64), frames).numpy()
    assert np.array_equal(got, np.repeat(x, dur, 0))
    gb = rng.standard_normal(2 * 512).astype(np.float32)
    y = rng.standard_normal((t, 512)).astype(np.float32)
    ref = (1 + gb[:512]) * F.layer_norm(torch.from_numpy(y).double(), (512,), eps=1e-5).numpy() + gb[512:]
    close(lk.ops.adalayernorm_f32_gpu(G(lk, y), G(lk, gb)), ref, 2e-5)
    v = rng.standard_normal(128).astype(np.float32)
    out = lk.ops.concat_bcast_f32_gpu(G(lk, y), G(lk, v)).numpy()
    assert np.array_equal(out, np.concatenate([y, np.broadcast_to(v, (t, 128))], 1))


# 4888: the 487-token forward's frames; 16500: past the LDS-staged phase scan's 16384 frames (the global-memory scan)
@pytest.mark.parametrize("n,voiced", [(574, True), (574, False), (4888, True), (16500, True)])
def test_harmonic_source_matches_f32_restatement(gpu, n, voiced):
    lk = gpu
    f0 = (150 + 20 * rng.standard_normal(n) if voiced else rng.standard_normal(n)).astype(np.float32)
    f0[:7] = 0.0  # unvoiced frames inside a voiced curve
    noise = rng.standard_normal((300 * n, 9)).astype(np.float32)
    w, b = (rng.standard_normal(9) / 3).astype(np.float32), np.array([0.05], np.float32)
    ref = OK.harmonic_source(f0, noise, w, b)
    got = lk.ops.harmonic_source_f32_gpu(G(lk, f0), G(lk, noise), G(lk, w), G(lk, b)).numpy()
    err = np.abs(got.astype(np.float64) - ref).max()
    assert err <= 2e-6, err  # same f32 phases: only sin / tanh ulps differ


@pytest.mark.parametrize("s", [3000, 172200])
def test_stft_magphase(gpu, s):
    lk = gpu
    x = np.tanh(rng.standard_normal(s) * 0.3).astype(np.float32)
    got = lk.ops.stft_magphase_lc_f32_gpu(G(lk, x)).numpy()
    z = torch.stft(torch.from_numpy(x).double(), 20, 5, 20, window=torch.hann_window(20, periodic=True,
                   dtype=torch.float64), center=True, pad_mode="reflect", return_complex=True)
    mag, ph = z.abs().numpy().T, torch.angle(z).numpy().T
    assert got.shape == (s // 5 + 1, 32) and not got[:, 22:].any()
    close(got[:, :11], mag, 2e-6)
    d = np.angle(np.exp(1j * (got[:, 11:22] - ph)))  # wrap-aware phase difference
    big = mag > 1e-3
    assert np.abs(d[big]).max() < 1e-3


def test_conv1d_1ch(gpu):
    lk = gpu
    x, w, b = rng.standard_normal(574).astype(np.float32), rng.standard_normal(3).astype(np.float32), np.float32([0.3])
    ref = F.conv1d(torch.from_numpy(x).double()[None, None], torch.from_numpy(w).double()[None, None],
                   torch.from_numpy(b).double(), stride=2, padding=1)[0, 0].numpy()
    close(lk.ops.conv1d_1ch_f32_gpu(G(lk, x), G(lk, w), G(lk, b), stride=2, padding=1), ref, 1e-6)
