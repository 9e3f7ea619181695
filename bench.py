"""Benchmark of the reference's headline metric on one MI355X:
"median Kokoro-82M f32 forward ms @59 & 487 tok; GPT-2 decode ms/token".

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload gpt2|kokoro487|kokoro59|all]

Prints ONE JSON line. `value` is the workload's median ms per step (lower is better) with inputs resident in
HBM; a "step" is one forward (Kokoro) or one decode step (GPT-2), replayed from its captured HIP graph.
`roofline` is the dominant kernel's algorithmic bytes or FLOPs per launch over its average launch time (HIP
events on the launch stream, standalone launches at the model's shape); `cpu_baseline` is the oracle's PyTorch
f32 CPU path timed on this host on a bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time

import numpy as np
import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
# HBM bytes one GPT-2 decode step at pos 512 must read: per layer the 4 weight matrices, their biases and the two
# LayerNorms; the tied LM head (wte); ln_f; the token and position rows; K and V rows 0..512 of 12 layers (f32)
GPT2_STEP_BYTES = 4 * (12 * (768 * 2304 + 768 * 768 + 2 * 768 * 3072 + 2304 + 768 + 3072 + 768 + 4 * 768)
                       + 50257 * 768 + 2 * 768 + 2 * 768 + 12 * 2 * 513 * 768)
F32_MFMA_PEAK_TFLOPS = 157.3


def event_times(fn, n: int) -> list[float]:
    """Per-call milliseconds of fn() measured with events on the current stream."""
    s = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for a, b in evs:
        a.record(s)
        fn()
        b.record(s)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in evs]


# ---- GPT-2 decode ---------------------------------------------------------------------------------------------

# algorithmic flops of the 512-token prefill: 12 layers x 2 x 512 x (768 x 2304 + 768 x 768 + 2 x 768 x 3072)
# for the projections, causal attention 12 layers x 12 heads x 2 x 2 x 64 x (512 x 513 / 2), LM head on the last row
PREFILL512_FLOPS = 12 * 2 * 512 * (768 * 2304 + 768 * 768 + 2 * 768 * 3072) + 12 * 12 * 4 * 64 * (512 * 513 // 2) \
    + 2 * 768 * 50257


def bench_gpt2(steps: int, warmup: int, cpu: bool = True) -> dict:
    import lokinfer_amd as lk
    from lokinfer_amd import gpt2 as G
    from oracle import gpt2 as O

    sd = G.random_weights()
    ids, nxt = O.decode_inputs()
    dec = G.Gpt2Generator(sd, chunk_graph=True)
    dec.prefill(ids)  # one 512-token chunk forward at pos 0
    # prefill of the 512-token prompt (captured chunk forward; rerunning it at pos 0 rewrites the same cache rows)
    pids = lk.from_numpy(ids, device="gpu", copy=True)
    pre = event_times(lambda: dec.run(pids, 0), 20)
    # a serving loop writes the step's token and position into the decoder's own input buffers (no copy per step)
    tok, pos = dec.tok, dec.pos
    tok.t.fill_(int(nxt))
    pos.t.fill_(512)
    for _ in range(warmup):
        dec.step(tok, pos)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dec.step(tok, pos)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    per = event_times(lambda: dec.step(tok, pos), max(steps, 20))
    # dominant kernel: the step's tail op (ln_f + tied LM head + argmax: lmHeadLnKernel, one wave per 4-row half
    # over wte, then the one-workgroup pass over the per-workgroup (max, index) pairs); 50257 x 768 f32 = 154.4 MB
    rng = np.random.default_rng(0)
    part = lk.from_numpy(rng.standard_normal((12, 768)).astype(np.float32), device="gpu", copy=True)
    vec = lambda: lk.from_numpy(rng.standard_normal(768).astype(np.float32), device="gpu", copy=True)  # noqa: E731
    bias, gamma, beta = vec(), vec(), vec()
    res = lk.from_numpy(rng.standard_normal((1, 768)).astype(np.float32), device="gpu", copy=True)
    wte = dec.w["transformer.wte.weight"]
    tables = [wte] + [lk.Tensor(wte.t.clone()) for _ in range(2)]  # 463 MB in turn: every call reads HBM
    kt = graph_ms([lambda t=t: lk.ops.lm_head_ln_argmax_f32_gpu(part, bias, res, gamma, beta, t) for t in tables])
    del tables
    lm_bytes = 50257 * 768 * 4 + (12 + 5) * 768 * 4 + 50257 * 4
    res = {
        "median_ms": statistics.median(per), "wall_ms_per_step": wall_ms,
        "roofline": {"kernel": "lmHeadLnKernel<3> + argmax pass (lm_head_ln_argmax_f32_gpu: ln_f, tied LM head, "
                               "argmax)", "bound": "hbm",
                     "achieved": lm_bytes / (kt * 1e-3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": lm_bytes / (kt * 1e-3) / 1e9 / HBM_PEAK_GBS, "traffic": None,
                     "avg_launch_ms": kt, "bytes_per_launch": lm_bytes},
        "step_bytes": GPT2_STEP_BYTES,
        "prefill512_ms": statistics.median(pre),
        "prefill512_tflops": PREFILL512_FLOPS / (statistics.median(pre) * 1e-3) / 1e12,
    }
    if cpu:
        res["cpu_baseline"] = cpu_gpt2(sd, ids, nxt)
    return res


def graph_ms(fn, n: int = 21, reps: int = 7) -> float:
    """Milliseconds per call of fn() replayed n times from one captured graph (median over reps replays): the
    device time per call, launch gaps included, without the host's per-call cost. fn may be a list of functions,
    called in turn (operands rotated through more memory than the 256 MB last-level cache holds)."""
    fns = fn if isinstance(fn, (list, tuple)) else [fn]
    for f in fns:
        f()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st = torch.cuda.Stream()
    with torch.cuda.stream(st):
        fns[0]()
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=st):
            for i in range(n):
                fns[i % len(fns)]()
    times = []
    for _ in range(reps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) / n)
    del g
    return statistics.median(times)


def bench_decode_attention() -> dict:
    """Decode attention against its HBM roofline: bytes = the K and V rows read, 2 (pos + 1) D x element size,
    over the per-call time of the kernel(s) replayed from a graph, with the calls rotated over enough cache copies
    (> 400 MB) that every call reads HBM, as in a decode step whose weight stream evicts the caches. Cases: the
    GPT-2 step's chunk kernel (attention_decode_part_f32_gpu: q / k / v from GEMV partials, 12 heads, 1024-row
    caches) at pos 512 and 1023; the split decode attention (attention_decode_split_f32_gpu: chunk + merge
    launches) on a 32768-row cache, where the K / V stream is long enough to be bandwidth-bound; Qwen3's f16 GQA
    decode (attention_gqa_opt_f16_gpu, 16 / 8 heads x 128) at its config-5 position 416 and on a 32768-row cache."""
    import lokinfer_amd as lk
    from lokinfer_amd import f16_gpu as F

    dev = torch.device("cuda")
    gen = torch.Generator(device=dev).manual_seed(0)
    T = lambda *shape, dt=torch.float32: lk.Tensor(torch.randn(*shape, device=dev, generator=gen).to(dt))  # noqa
    P = lambda v: lk.Tensor(torch.tensor([v], dtype=torch.int64, device=dev))  # noqa: E731
    out = {}

    def case(name, make, call, pos, cap, d, elem):
        nbytes = 2 * (pos + 1) * d * elem
        copies = max(1, -(-400_000_000 // (2 * cap * d * elem)))
        caches = [make() for _ in range(copies)]
        ms = graph_ms([lambda c=c: call(*c) for c in caches], n=max(21, copies))
        del caches
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[name] = {"us_per_call": round(ms * 1e3, 2), "bytes": nbytes, "achieved_gbs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4)}

    heads, d = 12, 768
    qp, qkv, bias = T(12, 3 * d), T(1, 3 * d), T(3 * d)
    for pos in (512, 1023):
        pt = P(pos)
        case(f"gpt2_step_chunk_pos{pos}", lambda: (T(1024, d), T(1024, d)),
             lambda kc, vc, pt=pt: lk.ops.attention_decode_part_f32_gpu(qp, kc, vc, pt, bias, heads), pos, 1024, d, 4)
    cap = 32768
    pt = P(cap - 1)
    case(f"split_f32_pos{cap - 1}", lambda: (T(cap, d), T(cap, d)),
         lambda kc, vc: lk.ops.attention_decode_split_f32_gpu(qkv, kc, vc, pt, bias, heads), cap - 1, cap, d, 4)
    q = T(1, 2048, dt=torch.float16)
    for cap, pos in ((480, 416), (32768, 32767)):
        pt = P(pos)
        case(f"qwen3_gqa_f16_pos{pos}", lambda cap=cap: (T(cap, 1024, dt=torch.float16), T(cap, 1024, dt=torch.float16)),
             lambda kc, vc, pt=pt: F.attention_gqa_opt_f16_gpu(q, kc, vc, pt, q_heads=16, kv_heads=8), pos, cap, 1024, 2)
    return out


def cpu_gpt2(sd, ids, nxt, budget_s: float = 15.0) -> dict:
    from oracle import gpt2 as O

    torch.set_num_threads(os.cpu_count() or 1)
    m = O.model(sd)
    past = O.prefill(m, ids)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end and len(times) < 200:
        t0 = time.perf_counter()
        _, past = O.decode_step(m, past, nxt)
        times.append((time.perf_counter() - t0) * 1e3)
        past.crop(512)
    return {"value": statistics.median(times[1:] or times), "unit": "ms/token", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"{len(times)} decode steps at pos 512 (transformers GPT2LMHeadModel f32, "
                                      f"same seeded weights), median"}


# ---- Kokoro-82M forward ----------------------------------------------------------------------------------------

def kokoro_conv_flops(tokens: int, frames: int) -> float:
    """Algorithmic (direct-convolution) FLOPs of one forward's convs + GEMMs, from the module shapes."""
    from lokinfer_amd import kokoro_weights as KW

    f, t = frames, tokens
    l0, l1 = 20 * f, 120 * f + 1
    mac = 0
    # ALBERT (12 layers) + bert_encoder
    mac += t * 128 * 768 + 12 * (t * 768 * 2304 + 2 * t * t * 768 + t * 768 * 768 + 2 * t * 768 * 2048) + t * 768 * 512
    # LSTM input projections (gate GEMMs) + recurrences: 3 duration-encoder + text encoder over T, shared over F
    mac += 3 * t * (640 * 2048 + 256 * 2048) + t * (512 * 2048 + 256 * 2048) + f * (640 * 2048 + 256 * 2048)
    # F0 / N: blocks 0 (512->512 @F), 1 (512->256 @2F + 1x1), 2 (256->256 @2F)
    mac += 2 * (2 * f * 512 * 512 * 3 + 2 * f * (512 * 256 * 3 + 256 * 256 * 3 + 512 * 256) + 2 * 2 * f * 256 * 256 * 3)
    # text encoder convs
    mac += 3 * t * 512 * 512 * 5
    # decoder: encode (514->1024 + 1x1), 3 decode (1090->1024 + 1x1), decode.3 (1090->512 @2F, 1x1), asr_res
    mac += f * (514 * 1024 * 3 + 1024 * 1024 * 3 + 514 * 1024) + 3 * f * (1090 * 1024 * 3 + 1024 * 1024 * 3 + 1090 * 1024)
    mac += 2 * f * (1090 * 512 * 3 + 512 * 512 * 3 + 1090 * 512) + f * 512 * 64
    # generator: noise convs, noise_res, ups (GEMM), resblocks, conv_post
    mac += l0 * 22 * 256 * 12 + l1 * 22 * 128
    mac += 6 * l0 * 256 * 256 * 7 + 6 * l1 * 128 * 128 * 11
    mac += 2 * f * 512 * 20 * 256 + l0 * 256 * 12 * 128
    mac += 6 * l0 * 256 * 256 * (3 + 7 + 11) + 6 * l1 * 128 * 128 * (3 + 7 + 11)
    mac += l1 * 128 * 22 * 7
    del KW
    return 2.0 * mac


def bench_kokoro(tokens: int, steps: int, warmup: int, runtime: str = "compiled", sd=None) -> dict:
    """Median ms of one Kokoro forward. runtime "compiled": lk.compile's C++ executable (one model arena, weights
    uploaded once, the call replayed from its captured hipGraph with the independent branches on 6 lanes);
    "capture": the torch stream capture of the same function."""
    import lokinfer_amd as lk
    from lokinfer_amd import kokoro_weights as KW
    from lokinfer_amd.kokoro import KokoroGpu

    sd = KW.random_weights() if sd is None else sd
    ids, ref_s, dur, noise = KW.inputs(tokens)
    frames = int(dur.sum())
    m = KokoroGpu(sd, runtime=runtime, lanes=6)
    args = [lk.from_numpy(a, device="gpu", copy=True) for a in (ids, ref_s, dur, noise)]
    for _ in range(max(warmup, 1)):
        m.forward(*args, inplace=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        m.forward(*args, inplace=True)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    model = m.model if runtime == "capture" else m.compiled(args)
    per = event_times(lambda: model.run_inplace(*args), steps)
    # A persistent kernel that stops on its bounded wait writes NaN; a timed run with such a launch is void.
    outs = model.run_inplace(*args)
    for o in (outs if isinstance(outs, tuple) else (outs,)):
        if not bool(torch.isfinite(o.t).all()):
            raise RuntimeError("kokoro forward produced non-finite outputs; timing discarded")
    return {"median_ms": statistics.median(per), "wall_ms_per_step": wall, "frames": frames,
            "flops": kokoro_conv_flops(tokens, frames), "sd": sd, "inputs": (ids, ref_s, dur, noise)}


ROOFLINE_SHAPE = (293281, 128, 11, 5)  # L = 120 F + 1 at 487 tokens (F = 2444), C = 128, K = 11, dilation 5
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "wino_mm_k11_L293281_traffic.txt")


def measured_traffic() -> float | None:
    """HBM bytes per launch of the roofline kernel from the committed rocprofv3 --pmc summary (FETCH_SIZE +
    WRITE_SIZE, calibrated against a copy kernel of known size), or None when it has not been measured."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def wino_tiles(lo: int, d: int, m: int = 4) -> int:
    """Output tiles of a dilated Winograd conv: sum over residue classes of ceil(rows / M)."""
    return sum(-(-len(range(r, lo, d)) // m) for r in range(d))


def roofline_wino(launches: int = 20, calibrate: bool = False) -> dict:
    """The dominant kernel of the Kokoro forward: the Winograd GEMM (winoMmKernel<4,7,3,3>, wino_mm_lc_f32_gpu with
    U tiled, u_layout 1, as the Kokoro graph runs it) of a generator stage-1 resblock conv (L = 120 F + 1 rows at 487 tokens, 128 -> 128 channels, K = 11 as 3 nested
    F(4,4) tap groups, d = 5). Its algorithm is A = 7 point GEMMs over (group, channel): 2 A T (N Ci) Co FLOPs
    per launch for T output tiles of 4 rows. The whole conv (input transform + GEMM, snake prologue) is timed
    beside it and reported against the direct conv's 2 L Ci Co K FLOPs. With calibrate, also launches add_f32_gpu
    over 2^26 floats (reads 512 MiB, writes 256 MiB) as the reference kernel for the --pmc byte counters."""
    import lokinfer_amd as lk
    from lokinfer_amd import winograd as W

    rng = np.random.default_rng(0)
    l, c, k, d = ROOFLINE_SHAPE
    pad = d * (k - 1) // 2
    G = lambda a: lk.from_numpy(np.ascontiguousarray(a, np.float32), device="gpu", copy=True)  # noqa: E731
    u, tr = W.wino_weights_t(rng.standard_normal((c, c, k)) / np.sqrt(c * k))
    x, u, tr, b = G(rng.standard_normal((l, c))), G(u), G(tr), G(rng.standard_normal(c))
    af = G(np.stack([np.zeros(c), np.ones(c), np.zeros(c)]))
    alpha = G(np.ones(c))
    _, n = W.variant(k)
    attrs = dict(dilation=d, groups=n, kernel=k, padding=pad, tile=4)
    v = lk.ops.wino_tf_lc_f32_gpu(x, tr, affine=af, alpha=alpha, **attrs)
    mm = lambda: lk.ops.wino_mm_lc_f32_gpu(v, u, b, tr, x, u_layout=1, **attrs)  # noqa: E731
    conv = lambda: lk.ops.conv1d_wino_lc_f32_gpu(x, u, b, tr, k, padding=pad, dilation=d, affine=af,  # noqa: E731
                                                 alpha=alpha, u_layout=1)
    mm()
    ms = statistics.mean(event_times(mm, launches))
    conv()
    conv_ms = statistics.mean(event_times(conv, max(5, launches // 2)))
    if calibrate:
        q = 1 << 26
        p1 = lk.Tensor(torch.ones(q, device="cuda"))
        p2 = lk.Tensor(torch.ones(q, device="cuda"))
        for _ in range(5):
            lk.ops.add_f32_gpu(p1, p2)
        torch.cuda.synchronize()
    a = W.alpha_of(k)
    flops = 2.0 * a * wino_tiles(l, d) * (n * c) * c
    direct = 2.0 * l * c * c * k
    return {"kernel": "winoMmKernel<4,7,3,3,1,true> (wino_mm_lc_f32_gpu, tiled U: K = 11 Winograd GEMM, "
                      "generator stage 1)",
            "bound": "mfma", "achieved": flops / (ms * 1e-3) / 1e12, "peak": F32_MFMA_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": flops / (ms * 1e-3) / 1e12 / F32_MFMA_PEAK_TFLOPS,
            "traffic": measured_traffic(), "avg_launch_ms": ms, "flops_per_launch": flops,
            "conv_ms": conv_ms, "conv_direct_equiv_tflops": direct / (conv_ms * 1e-3) / 1e12}


def cpu_kokoro(sd, inputs, budget_s: float = 30.0) -> dict:
    from oracle.kokoro import Oracle

    torch.set_num_threads(os.cpu_count() or 1)
    o = Oracle(sd)
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (time.perf_counter() < t_end and len(times) < 3):
        t0 = time.perf_counter()
        o.forward(*inputs)
        times.append((time.perf_counter() - t0) * 1e3)
    return {"value": statistics.median(times), "unit": "ms", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"{len(times)} full forward(s) of the same {len(inputs[0])}-token config (PyTorch f32 CPU "
                      f"restatement of the Kokoro-82M graph, same weights and inputs), median"}


# ---- Qwen3-ASR LM f16 (config 5) -----------------------------------------------------------------------------

def bench_qwen3(steps: int, warmup: int) -> dict:
    """Config 5: prefill of 16 prompt ids + 400 audio rows (T = 416, one chunk at pos 0), then decode steps at
    pos 416.. (one captured graph), f16 weights and caller-owned f16 KV cache resident in HBM."""
    from lokinfer_amd import qwen3 as M

    cfg = M.CONFIG5
    sd = M.random_weights(cfg)
    ids, audio = M.config5_inputs(cfg)
    lm = M.Qwen3Lm(sd, cfg)
    del sd
    kv = lm.kv_cache(len(ids) + 64)
    ids_d = lm._dev(ids, np.int64)
    audio_d = lm._dev(audio, np.float16)
    lm.run(ids_d, audio_d, 0, kv)  # captures the prefill graph
    pre = event_times(lambda: lm.run(ids_d, audio_d, 0, kv), max(5, steps // 4))
    tok = lm._dev(np.array([1000], np.int64), np.int64)
    dummy = lm._dev(np.zeros((1, cfg.d), np.float16), np.float16)
    pos = len(ids)
    for _ in range(warmup):
        lm.run(tok, dummy, pos, kv)
    dec = event_times(lambda: lm.run(tok, dummy, pos, kv), steps)
    wbytes = sum(L["qkv"].wt.nbytes + L["gateup"].wt.nbytes + L["o"].wt.nbytes + L["down"].wt.nbytes
                 for L in lm.layers) + lm.embed.nbytes
    kvbytes = cfg.layers * 2 * (pos + 1) * cfg.dk * 2
    flops = 2 * len(ids) * cfg.layers * (cfg.d * (cfg.dq + 2 * cfg.dk) + cfg.dq * cfg.d + 3 * cfg.d * cfg.ffn)
    dm = statistics.median(dec)
    return {"prefill_ms": statistics.median(pre), "prefill_tflops": flops / (statistics.median(pre) * 1e-3) / 1e12,
            "decode_ms": dm, "decode_bytes": wbytes + kvbytes,
            "decode_hbm_gbs": (wbytes + kvbytes) / (dm * 1e-3) / 1e9}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="all", choices=["all", "kokoro487", "kokoro59", "gpt2", "qwen3", "decode_attn"])
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--runtime", default="compiled", choices=["compiled", "capture"],
                    help="Kokoro: the lk.compile C++ executable (default) or the torch stream capture")
    ap.add_argument("--roofline-only", action="store_true",
                    help="launch only the roofline kernel (and the copy-calibration kernel), for rocprofv3 runs")
    a = ap.parse_args()
    if a.roofline_only:
        r = roofline_wino(launches=a.steps, calibrate=True)
        print(json.dumps({k: v for k, v in r.items()}))
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this backend has no multi-GPU path (every box has one GPU)",
              file=sys.stderr)
        sys.exit(2)
    wl = a.workload
    if wl == "qwen3":  # config 5 (not in the headline metric): prefill + decode of the f16 LM
        r = bench_qwen3(a.steps, a.warmup)
        line = {
            "metric": "Qwen3-ASR LM f16 decode ms/token (config 5; not the headline metric)",
            "value": round(r["decode_ms"], 4), "unit": "ms/token", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
            "ms_per_step": round(r["decode_ms"], 4), "higher_is_better": False, "scaling": "weak",
            "vs_baseline": None, "dtype": "f16", "data": "synthetic (seeded random-init weights, ids, audio rows)",
            "config": {"workload": "qwen3-asr LM 28 layers, 416-id prefill (400 audio rows), decode at pos 416",
                       "model": "qwen3-asr-1.7b-lm", "global_batch": 1, "seq_len": 417, "parallelism": "none"},
            "roofline": {"bound": "hbm", "achieved": round(r["decode_hbm_gbs"], 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(r["decode_hbm_gbs"] / HBM_PEAK_GBS, 4), "traffic": None},
            "decode_bytes_per_token": r["decode_bytes"],
            "prefill416_ms": round(r["prefill_ms"], 3), "prefill416_tflops": round(r["prefill_tflops"], 1),
            "cpu_baseline": None,
        }
        print(json.dumps(line))
        return
    if wl == "gpt2":
        r = bench_gpt2(a.steps, a.warmup, cpu=not a.no_cpu)
        line = {
            "metric": "median Kokoro-82M f32 forward ms @59 & 487 tok; GPT-2 decode ms/token",
            "value": round(r["median_ms"], 4), "unit": "ms/token", "n_gpus": 1, "steps": a.steps,
            "warmup": a.warmup, "ms_per_step": round(r["wall_ms_per_step"], 4), "higher_is_better": False,
            "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (seeded random-init weights and token ids)",
            "config": {"workload": "gpt2-124m decode 1 token @ 512 cached, batch 1", "model": "gpt2-124m",
                       "global_batch": 1, "seq_len": 513, "parallelism": "none"},
            "roofline": {k: r["roofline"][k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")},
            "roofline_kernel": r["roofline"]["kernel"], "cpu_baseline": r.get("cpu_baseline"),
            "gpt2_prefill512_ms": round(r["prefill512_ms"], 4),
            "gpt2_prefill512_tflops": round(r["prefill512_tflops"], 2),
            "gpt2_step_hbm_frac": round(GPT2_STEP_BYTES / (r["median_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "decode_attention_roofline": bench_decode_attention(),
        }
        print(json.dumps(line))
        return
    if wl == "decode_attn":  # the decode-attention leg alone (for rocprofv3 runs)
        print(json.dumps({"decode_attention_roofline": bench_decode_attention()}))
        return
    tokens = 59 if wl == "kokoro59" else 487
    r = bench_kokoro(tokens, a.steps, a.warmup, runtime=a.runtime)
    extra = {"runtime": a.runtime}
    if wl == "all":
        other = "capture" if a.runtime == "compiled" else "compiled"
        extra[f"kokoro{tokens}_{other}_ms"] = round(bench_kokoro(tokens, a.steps, a.warmup, other, r["sd"])["median_ms"], 3)
        r59 = bench_kokoro(59, a.steps, a.warmup, a.runtime, r["sd"])
        g = bench_gpt2(max(a.steps, 20), a.warmup, cpu=not a.no_cpu)
        extra.update({"kokoro59_median_ms": round(r59["median_ms"], 3), "kokoro59_frames": r59["frames"],
                 "kokoro59_cpu_baseline": None if a.no_cpu else cpu_kokoro(r59["sd"], r59["inputs"], budget_s=10.0),
                 "gpt2_decode_median_ms": round(g["median_ms"], 4), "gpt2_decode_cpu_baseline": g.get("cpu_baseline"),
                 "gpt2_step_hbm_frac": round(GPT2_STEP_BYTES / (g["median_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                 "gpt2_lm_head_roofline": g["roofline"],
                 "gpt2_prefill512_ms": round(g["prefill512_ms"], 4),
                 "gpt2_prefill512_tflops": round(g["prefill512_tflops"], 2),
                 "decode_attention_roofline": bench_decode_attention()})
    roof = roofline_wino()
    cpu = None if a.no_cpu else cpu_kokoro(r["sd"], r["inputs"])
    line = {
        "metric": "median Kokoro-82M f32 forward ms @59 & 487 tok; GPT-2 decode ms/token",
        "value": round(r["median_ms"], 3), "unit": "ms", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(r["wall_ms_per_step"], 3), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded random-init Kokoro-82M-shaped weights, ids, style, durations 2..8, noise)",
        "config": {"workload": f"kokoro-82m forward, {tokens} tokens, {r['frames']} frames "
                               f"({600 * r['frames']} samples), forced durations", "model": "kokoro-82m",
                   "global_batch": 1, "seq_len": tokens, "parallelism": "none"},
        "roofline": {k: roof[k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")},
        "roofline_kernel": roof["kernel"], "roofline_avg_launch_ms": roof["avg_launch_ms"],
        "roofline_conv_ms": roof["conv_ms"], "roofline_conv_direct_equiv_tflops": roof["conv_direct_equiv_tflops"],
        "forward_algorithmic_tflops": round(r["flops"] / (r["median_ms"] * 1e-3) / 1e12, 2),
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
