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

def bench_gpt2(steps: int, warmup: int, cpu: bool = True) -> dict:
    import lokinfer_amd as lk
    from lokinfer_amd import gpt2 as G
    from oracle import gpt2 as O

    sd = G.random_weights()
    ids, nxt = O.decode_inputs()
    dec = G.Gpt2Decoder(sd)
    dec.prefill(ids)
    tok = lk.from_numpy(np.array([nxt], np.int64), device="gpu", copy=True)
    pos = lk.from_numpy(np.array([512], np.int64), device="gpu", copy=True)
    for _ in range(warmup):
        dec.step(tok, pos)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        dec.step(tok, pos)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    per = event_times(lambda: dec.step(tok, pos), max(steps, 20))
    # dominant kernel: the tied LM head (gemm_nt at M = 1: one wave per wte row), 50257 x 768 f32 = 154.4 MB
    ln = lk.from_numpy(np.random.default_rng(0).standard_normal((1, 768)).astype(np.float32), device="gpu")
    wte = dec.w["transformer.wte.weight"]
    lk.ops.gemm_nt_f32_gpu_mps(ln, wte)
    kt = statistics.mean(event_times(lambda: lk.ops.gemm_nt_f32_gpu_mps(ln, wte), 50))
    lm_bytes = 50257 * 768 * 4 + 768 * 4 + 50257 * 4
    res = {
        "median_ms": statistics.median(per), "wall_ms_per_step": wall_ms,
        "roofline": {"kernel": "rowdotKernel<1> (gemm_nt_f32_gpu_mps, LM head)", "bound": "hbm",
                     "achieved": lm_bytes / (kt * 1e-3) / 1e9, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": lm_bytes / (kt * 1e-3) / 1e9 / HBM_PEAK_GBS, "traffic": None,
                     "avg_launch_ms": kt, "bytes_per_launch": lm_bytes},
        "step_bytes": 532.4e6,
    }
    if cpu:
        res["cpu_baseline"] = cpu_gpt2(sd, ids, nxt)
    return res


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="gpt2")
    ap.add_argument("--no-cpu", action="store_true")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this backend has no multi-GPU path (every box has one GPU)",
              file=sys.stderr)
        sys.exit(2)
    r = bench_gpt2(a.steps, a.warmup, cpu=not a.no_cpu)
    line = {
        "metric": "median Kokoro-82M f32 forward ms @59 & 487 tok; GPT-2 decode ms/token",
        "value": round(r["median_ms"], 4), "unit": "ms/token", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(r["wall_ms_per_step"], 4), "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic (seeded random-init weights and token ids)",
        "config": {"workload": "gpt2-124m decode 1 token @ 512 cached, batch 1", "model": "gpt2-124m",
                   "global_batch": 1, "seq_len": 513, "parallelism": "none"},
        "roofline": {k: r["roofline"][k] for k in ("bound", "achieved", "peak", "unit", "frac", "traffic")},
        "roofline_kernel": r["roofline"]["kernel"], "roofline_avg_launch_ms": r["roofline"]["avg_launch_ms"],
        "cpu_baseline": r.get("cpu_baseline"),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
