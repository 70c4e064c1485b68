#!/usr/bin/env python3
"""Throughput of the LoRA-MoE ChannelMix forward on one MI355X.

A step is one forward of the D=768, F=3072, E=8, top-2, r=16 fp16 layer over
8 x 512 = 4096 tokens (the 184M-model layer shape), inputs resident in HBM.
Prints one JSON line: whole-layer tokens/s, the roofline of the dominant
kernel (timed live with HIP events on the launch stream) and a CPU baseline
(the NumPy restatement of the reference algorithm on a bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "rwkv-mlx_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "MoE-ChannelMix tokens/s + %HBM/%MFMA roofline, D768 E8 top-2 r16 fp16"
PEAK_MFMA_F16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=["fused", "sparse"], default="fused")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget for the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--kernels-only", action="store_true", help="also print a per-stage timing table to stderr")
    return ap.parse_args()


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this build measures one GPU only: the forward runs on a single MI355X and "
                                   "no multi-GPU path is built; run with --gpus 1"}))
        sys.exit(2)

    import numpy as np
    import torch

    from rwkv_mlx_amd import _lib
    from rwkv_mlx_amd.workloads import HEADLINE, make_inputs

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    w = HEADLINE
    N, C, F, E, k, r = w.tokens, w.d_model, w.d_ffn, w.n_experts, w.top_k, w.lora_rank
    g = make_inputs(w)
    dt = torch.float16

    def up(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dt)

    x, xk, Wk, Wv, Wg, A, B = (up(g[n]) for n in ("x", "x_k", "Wk", "Wv", "Wg", "A", "B"))
    out = torch.empty_like(x)
    losses = torch.empty(2, dtype=torch.float32, device=dev)
    desc = _lib.make_desc(w.batch, w.seq_len, C, F, E, k, r, "f16", args.mode)
    nbytes = _lib.workspace_bytes(desc)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    fwd = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, w_value=Wv, w_gate=Wg, lora_A=A, lora_B=B, out=out,
                            losses=losses)

    def step():
        _lib.call("rwkvmoe_forward", desc, fwd, ws, nbytes, sh)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / args.steps
    tokens_per_s = N / (ms * 1e-3)

    # ---- dominant kernels, each timed alone on the same stream ---------------
    hidden = torch.empty(N, F, dtype=dt, device=dev)
    base = torch.empty(N, C, dtype=dt, device=dev)
    key_t = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, hidden=hidden)
    val_t = _lib.make_tensors(hidden=hidden, w_value=Wv, base_out=base)

    def timed(fn, reps):
        for _ in range(5):
            fn()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            fn()
        b.record(stream)
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps * 1e3  # us

    reps = max(args.steps, 50)
    key_us = timed(lambda: _lib.call("rwkvmoe_cmix_key", desc, key_t, ws, nbytes, sh), reps)
    val_us = timed(lambda: _lib.call("rwkvmoe_cmix_value", desc, val_t, ws, nbytes, sh), reps)
    gemm_flop = 2.0 * N * C * F
    kern = {"cmix_key": key_us, "cmix_value": val_us}
    dom_name, dom_us = max(kern.items(), key=lambda kv: kv[1])
    achieved = gemm_flop / (dom_us * 1e-6) / 1e12
    roofline = {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_MFMA_F16_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_MFMA_F16_TFLOPS, 4), "traffic": None, "kernel": dom_name,
                "kernel_us": round(dom_us, 3), "algorithmic_flop": gemm_flop}
    if args.kernels_only:
        print(json.dumps({k2: round(v, 3) for k2, v in kern.items()}), file=sys.stderr)

    # ---- CPU baseline: the oracle's restatement of the reference algorithm ----
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w, g, args.cpu_seconds)

    rec = {
        "metric": METRIC, "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f16", "data": "synthetic (seeded N(0,1) inputs, "
        "reference-shaped random weights)",
        "config": {"workload": w.name, "tokens": N, "batch": w.batch, "seq_len": w.seq_len, "d_model": C,
                   "d_ffn": F, "n_experts": E, "top_k": k, "lora_rank": r, "mode": args.mode,
                   "parallelism": "single GPU"},
        "roofline": roofline, "cpu_baseline": cpu, "wall_s": round(wall, 4),
    }
    print(json.dumps(rec))


def cpu_baseline(w, g, budget_s):
    """Time the oracle (fp32 products) on one 512-token sequence of the layer,
    repeated within ``budget_s`` seconds; tokens/s scaled to the metric."""
    import numpy as np

    from oracle import moe_oracle as O
    try:
        from threadpoolctl import threadpool_info
        threads = max([i.get("num_threads", 1) for i in threadpool_info()] or [1])
    except Exception:
        threads = os.cpu_count() or 1
    T = w.seq_len
    xs = g["x"][:1]
    O.moe_forward(xs, g, w.top_k, w.dtype, mm_dtype=np.float32)  # warm-up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 2:
        t = time.perf_counter()
        O.moe_forward(xs, g, w.top_k, w.dtype, mm_dtype=np.float32)
        times.append(time.perf_counter() - t)
    med = float(np.median(times))
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"value": round(T / med, 1), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle moe_forward (NumPy, fp32 products, dense expert loop) on 1 x {T} tokens of the "
                      f"{w.name} layer, median of {len(times)} runs", "cpu_model": cpu_model}


if __name__ == "__main__":
    main()
