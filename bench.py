#!/usr/bin/env python3
"""Throughput of the LoRA-MoE ChannelMix forward on one MI355X.

A step is one forward of the D=768, F=3072, E=8, top-2, r=16 fp16 layer over
8 x 512 = 4096 tokens (the 184M-model layer shape), inputs resident in HBM.
The adapters are laid out once by rwkvmoe_prepare_adapters (as the torch
module caches them while they are unchanged), so a forward is the router,
the key GEMM and the value GEMM.
Prints one JSON line:
  * value: whole-layer tokens/s, from HIP events around K back-to-back
    forwards on one stream, after at least W untimed forwards and at least
    50 ms of them (the GPU's clocks settle over its first tens of
    milliseconds of work: the first 200 forwards of a fresh process average
    ~120 us against ~63 us in the steady state); a short spin kernel ahead
    of the first event holds the GPU while the host enqueues the first
    forwards, and the host stays ahead after that (~8 us to enqueue a
    forward), so the events see the GPU's pace and never the host's;
  * forward_unprepared: the same forward laying the adapters out itself
    (one more launch), and prepare_adapters_us, the layout pass alone;
  * kernels: every kernel of one forward over a second run of K forwards:
    `us`, the kernel's own duration from the begin / end timestamps its
    launch records (rwkvmoe_forward_timed with per-launch event pairs, the
    figure a kernel trace reports), with its algorithmic bytes or FLOPs and
    its fraction of the HBM or MFMA roofline; `us_marginal`, what it adds to
    a forward (its interval between events recorded on the stream, less what
    those records add around an empty kernel); the same table for the SPARSE
    mode (dispatch, grouped LoRA, combine);
  * roofline: the entry of the kernel that takes the most time per forward;
    `traffic` comes from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    counter summary of that kernel, and `rocprof` from the committed kernel
    trace of the workload (profiles/kernels_<workload>.json), when there is
    one;
  * graph_replay: the forward captured in HIP graphs, 10 forwards per graph
    (per-forward time) and one forward per graph;
  * single_forward: warm and cache-flushed medians of forwards timed one at
    a time (the flush is a 512 MB device write before each forward), with
    the per-kernel split of both;
  * sparse_forward: the same layer in SPARSE mode (dispatch, grouped LoRA,
    combine), timed like the headline;
  * mixed_forward: the reference's fine-tune form of the layer (fp16 x and
    base, fp32 router gate and adapters: RWKVMOE_GATE_F32 |
    RWKVMOE_ADAPTERS_F32, fp32 output), both modes, beside the fp16 layer;
  * block_forward: the Block's form x + ffn(ln2(x)) on the residual stream
    (RWKVMOE_LN_IN | RWKVMOE_ADD_RESIDUAL, residual = x), timed the same
    way, and its time over the layer's;
  * backward: the VJP (rwkvmoe_backward) timed the same way;
  * experts: the full-expert layer (MoE_CMix, rwkvmoe_experts_forward) of
    the same shape with random expert weights, timed the same way, and its
    VJP (rwkvmoe_experts_backward, every input and parameter);
  * cpu_baseline: the NumPy restatement of the reference algorithm (the
    literal dense expert loop) on a bounded sample, on this host's cores.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from dataclasses import replace
from pathlib import Path

REPO = Path(__file__).resolve().parent
for _p in (REPO, REPO / "rwkv-mlx_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "MoE-ChannelMix tokens/s + %HBM/%MFMA roofline, D768 E8 top-2 r16 fp16"
PEAK_MFMA_TFLOPS = {"f16": 2500.0, "bf16": 2500.0, "f32": 157.3}
PEAK_HBM_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--mode", choices=["fused", "sparse"], default="fused")
    from rwkv_mlx_amd.workloads import BY_NAME, HEADLINE
    ap.add_argument("--workload", choices=sorted(BY_NAME), default=HEADLINE.name,
                    help="layer shape (default: the D=768 E=8 top-2 r=16 fp16 layer the metric is quoted on; "
                         "the others are for per-kernel tables and profiles)")
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="budget for the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-kernels", action="store_true", help="skip the per-kernel tables")
    ap.add_argument("--no-backward", action="store_true", help="skip the backward (VJP) timing")
    ap.add_argument("--no-graph", action="store_true", help="skip the HIP graph replay timing")
    ap.add_argument("--vs-hipblaslt", action="store_true",
                    help="also time torch.matmul (hipBLASLt) on the layer's two plain products")
    ap.add_argument("--backward-only", action="store_true", help="time only the backward (for kernel traces)")
    ap.add_argument("--no-experts", action="store_true", help="skip the full-expert layer (MoE_CMix) timing")
    ap.add_argument("--experts-only", action="store_true", help="time only the full-expert layer (for kernel traces)")
    ap.add_argument("--mixed-only", action="store_true",
                    help="time only the fp16-base / fp32-adapter layer (for kernel traces)")
    ap.add_argument("--block-only", action="store_true",
                    help="time only the Block form x + ffn(ln2(x)) (for kernel traces)")
    ap.add_argument("--single", type=int, default=30, metavar="K",
                    help="forwards timed one at a time for the warm and cache-flushed medians (0: skip)")
    ap.add_argument("--table", action="store_true", help="also print the per-kernel tables to stderr")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB device-to-device 3 times (a plain copy kernel of known size, "
                         "to scale HBM byte counters)")
    return ap.parse_args()


def router_tile_tokens(w, s: int) -> int:
    """Tokens per router workgroup, as the library chooses them."""
    N, C, E = w.tokens, w.d_model, w.n_experts
    tt = min(16, 4096 // max(E * (C // 64), 1), 65536 // ((C + 16 // s) * s) - 2, -(-N // 64))
    return max(tt, 1)


def kernel_cost(name: str, w, kx: int, s: int, router_u: bool):
    """(bound, algorithmic amount, unit) of one launch of kernel `name` on
    layer `w`: bytes a fused kernel must move between HBM and the chip (its
    external inputs and outputs, each once), or the FLOPs of its product."""
    N, C, F, E, k, r = w.tokens, w.d_model, w.d_ffn, w.n_experts, w.top_k, w.lora_rank
    nbr = -(-N // router_tile_tokens(w, s))
    if name == "lora_prep":
        return "hbm", 2 * (E * C * r * s + kx * C * s), "B"
    if name == "router":
        b = N * C * s + E * C * s + C * s                     # x, W_gate, x_k
        b += N * k * 4 + N * k * s + N * E * s                # inds, gates, dense gates
        b += N * C * s                                        # xk
        b += nbr * ((E + 1) * 8 + E * 4)                      # loss partials
        if router_u:
            b += kx * C * s + N * kx * s                      # A_all in, U out
        return "hbm", b, "B"
    if name == "decode_front":
        # the router (no xk written), the key tiles (W_key and the shift
        # state in, hidden out) and the adapter tiles (A_all in, u out)
        _, b, _ = kernel_cost("router", w, kx, s, False)
        return "hbm", b - N * C * s + (F * C * s + N * C * s + N * F * s) + (kx * C * s + N * kx * s), "B"
    if name == "decode_value":
        # W_value and B_all in, hidden, u and the dense gates in, out (+ the losses)
        return "hbm", (C * F * s + C * kx * s + N * F * s + N * kx * s + N * E * s + N * C * s
                       + nbr * ((E + 1) * 8 + E * 4)), "B"
    if name == "router_finalize":
        return "hbm", nbr * ((E + 1) * 8 + E * 4) + 8, "B"
    if name == "shift_mix":
        return "hbm", 2 * N * C * s + C * s, "B"
    if name.startswith("cmix_key"):
        return "mfma", 2.0 * N * C * F, "FLOP"
    if name == "cmix_adapters":  # the adapter columns alone: U = w ⊙ (x · A_allᵀ)
        return "mfma", 2.0 * N * C * E * r, "FLOP"
    if name.startswith("cmix_value"):
        return "mfma", 2.0 * N * F * C, "FLOP"
    if name == "dispatch":
        return "hbm", N * k * 4 + N * k * 8 + (E + 1) * 4, "B"   # inds in; perm, inv_perm, offsets out
    if name == "dispatch_count":
        return "hbm", N * k * 4, "B"
    if name == "dispatch_scatter":
        return "hbm", N * k * 4 + N * k * 8 + (E + 1) * 4, "B"
    if name == "lora_grouped":
        return "hbm", 2 * N * k * C * s + 2 * E * C * r * s + N * k * 4, "B"
    if name == "combine":
        return "hbm", 2 * N * C * s + N * k * C * s + N * k * (4 + s + 4), "B"
    if name in ("ortho_pairs", "ortho_final"):
        return "hbm", E * C * r * s if name == "ortho_pairs" else 4, "B"
    return "hbm", 0, "B"


def kernel_table(timings, intervals, w, kx, s, dtype, router_u, overhead_us=0.0):
    """Per-kernel rows of one forward.  `us`: the kernel's own duration, from
    the begin / end timestamps its launch records (as a kernel trace reports
    it; the fixed cost at either end of a launch overlaps its neighbours in a
    back-to-back stream, so these can sum to more than a step); the roofline
    fraction follows from it.  `us_marginal`: what the kernel adds to a
    forward, its interval between events recorded on the stream less what
    those records add around an empty kernel (event_overhead_us)."""
    rows = []
    iv = dict(intervals)
    for name, us in timings:
        us_marg = max(iv.get(name, float("nan")) - overhead_us, 0.0)
        bound, amount, unit = kernel_cost(name, w, kx, s, router_u)
        if bound == "mfma":
            achieved, peak, u = amount / (us * 1e-6) / 1e12, PEAK_MFMA_TFLOPS[dtype], "TFLOP/s"
        else:
            achieved, peak, u = amount / (us * 1e-6) / 1e9, PEAK_HBM_GBS, "GB/s"
        rows.append({"kernel": name, "us": round(us, 3), "us_marginal": round(us_marg, 3), "bound": bound,
                     "algorithmic": amount,
                     "algorithmic_unit": unit, "achieved": round(achieved, 2), "peak": peak, "unit": u,
                     "frac": round(achieved / peak, 4)})
    return rows


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
    from rwkv_mlx_amd.workloads import BY_NAME, HEADLINE, make_inputs

    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.calibrate_copy > 0:
        src = torch.ones(args.calibrate_copy << 18, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    w = BY_NAME[args.workload]
    N, C, F, E, k, r = w.tokens, w.d_model, w.d_ffn, w.n_experts, w.top_k, w.lora_rank
    g = make_inputs(w)
    dt = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}[w.dtype]
    s = 4 if w.dtype == "f32" else 2
    kx = -(-E * r // 128) * 128

    def up(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dt)

    x, xk, Wk, Wv, Wg, A, B = (up(g[n]) for n in ("x", "x_k", "Wk", "Wv", "Wg", "A", "B"))
    out = torch.empty_like(x)
    losses = torch.empty(2, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    flags, extra = 0, {}
    if "x_prev" in g:  # decode step: the carried shift state
        flags |= _lib.HAS_PREV
        extra["x_prev"] = up(g["x_prev"])
    if "bias" in g:    # skewed routing: the Zipf logit bias
        flags |= _lib.HAS_BIAS
        extra["logit_bias"] = torch.from_numpy(g["bias"]).to(dev)
    def setup(mode):
        desc = _lib.make_desc(w.batch, w.seq_len, C, F, E, k, r, w.dtype, mode, flags)
        nbytes = _lib.workspace_bytes(desc)
        return desc, torch.empty(nbytes, dtype=torch.uint8, device=dev), nbytes

    desc, ws, nbytes = setup(args.mode)
    # the adapters' kernel layouts, made once (constant weights)
    prep = torch.empty(_lib.prepared_bytes(desc), dtype=torch.uint8, device=dev)
    _lib.prepare_adapters(desc, A, B, prep, sh)
    pbase = None
    if _lib.reads_prepared_base(desc):
        # decode-sized forwards read the frozen base W_key / W_value in the
        # decode launches' fragment order, also made once
        pbase = torch.empty(_lib.prepared_base_bytes(desc), dtype=torch.uint8, device=dev)
        _lib.prepare_base(desc, Wk, Wv, pbase, sh)
    fwd = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, w_value=Wv, w_gate=Wg, lora_A=A, lora_B=B, out=out,
                            losses=losses, prepared=prep, prepared_base=pbase, **extra)
    fwd_raw = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, w_value=Wv, w_gate=Wg, lora_A=A, lora_B=B, out=out,
                                losses=losses, **extra)
    # SPARSE with the adapter rows asked for: the dispatch / grouped LoRA /
    # combine form (the default SPARSE form keeps the adapters on chip where
    # the layer allows it)
    rows_buf = torch.empty(N * k, C, dtype=dt, device=dev)
    fwd_rows = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, w_value=Wv, w_gate=Wg, lora_A=A, lora_B=B, out=out,
                                 losses=losses, prepared=prep, prepared_base=pbase, adapter_rows=rows_buf, **extra)

    # at least 50 ms of forwards before anything is timed: the GPU's clocks
    # settle over its first tens of milliseconds of work
    warm_end = time.perf_counter() + 0.05
    while time.perf_counter() < warm_end:
        for _ in range(50):
            _lib.call("rwkvmoe_forward", desc, fwd, ws, nbytes, sh)
        torch.cuda.synchronize()

    # what the HIP events around each kernel add to its interval (subtracted
    # from every per-kernel figure below)
    overhead = event_overhead_us(stream)

    def time_loop(fn):
        """ms per call of fn over args.steps back-to-back calls after
        args.warmup untimed ones, HIP events on the stream."""
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        hold_queue()  # the host enqueues the timed calls while the GPU waits: the events see the GPU's pace
        e0.record(stream)
        for _ in range(args.steps):
            fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / args.steps

    def time_sparse():
        d2, ws2, nb2 = setup("sparse")
        sms = time_loop(lambda: _lib.call("rwkvmoe_forward", d2, fwd, ws2, nb2, sh))
        res = {"ms_per_step": round(sms, 5), "tokens_per_s": round(N / (sms * 1e-3), 1),
               "mode": "sparse: the adapters on chip (router u, the value product's rank slices) where E*r <= 128 "
                       "with 16-bit types, else dispatch, grouped LoRA over routed rows, combine"}
        # the dispatch / grouped LoRA / combine form (adapter rows asked for)
        gms = time_loop(lambda: _lib.call("rwkvmoe_forward", d2, fwd_rows, ws2, nb2, sh))
        res["grouped_forward"] = {"ms_per_step": round(gms, 5), "tokens_per_s": round(N / (gms * 1e-3), 1),
                                  "form": "dispatch, grouped LoRA over routed rows (adapter rows out), combine"}
        # the MFMA-or-VALU choice of the grouped LoRA: the same forward with
        # its products on the vector ALUs (RWKVMOE_LORA_VALU), and both forms'
        # grouped-LoRA kernel alone (event-timed on the stream)
        dv = _lib.make_desc(w.batch, w.seq_len, C, F, E, k, r, w.dtype, "sparse", flags | _lib.LORA_VALU)
        vms = time_loop(lambda: _lib.call("rwkvmoe_forward", dv, fwd, ws2, nb2, sh))
        res["lora_valu_forward"] = {"ms_per_step": round(vms, 5), "tokens_per_s": round(N / (vms * 1e-3), 1)}
        if not args.no_kernels:
            for label, dd in (("lora_grouped_mfma_us", d2), ("lora_grouped_valu_us", dv)):
                timer = _lib.KernelTimer(stream, args.steps)
                hold_queue()
                for _ in range(args.steps):
                    timer.forward(dd, fwd_rows, ws2, nb2)
                res[label] = round(dict(timer.summary()).get("lora_grouped", float("nan")), 3)
                del timer
        return res

    def time_block():
        """The Block's x + ffn(ln2(x)) (model.py:321-322): ln2 (seeded
        weight and bias) applied inside the forward, residual = x."""
        rng = np.random.default_rng(7)
        lw = up(1.0 + 0.1 * rng.standard_normal(C).astype(np.float32))
        lb = up(0.05 * rng.standard_normal(C).astype(np.float32))
        db = _lib.make_desc(w.batch, w.seq_len, C, F, E, k, r, w.dtype, args.mode,
                            flags | _lib.LN_IN | _lib.ADD_RESIDUAL)
        nbb = _lib.workspace_bytes(db)
        wsb = torch.empty(nbb, dtype=torch.uint8, device=dev)
        tb = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, w_value=Wv, w_gate=Wg, lora_A=A, lora_B=B, out=out,
                               losses=losses, prepared=prep, prepared_base=pbase, ln_weight=lw, ln_bias=lb,
                               residual=x, **extra)
        bms = time_loop(lambda: _lib.call("rwkvmoe_forward", db, tb, wsb, nbb, sh))
        return {"ms_per_step": round(bms, 5), "tokens_per_s": round(N / (bms * 1e-3), 1),
                "form": "x + ffn(ln2(x)) on the residual stream (RWKVMOE_LN_IN | RWKVMOE_ADD_RESIDUAL)"}

    def time_mixed():
        """fp16 x and base with fp32 W_gate, lora_A, lora_B (the layer
        finetune_moe.py trains on a converted fp16 checkpoint), both modes."""
        if w.dtype != "f16":
            return None
        f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
        gm = make_inputs(replace(w, dtype="f32"))
        Am, Bmx = f32(gm["A"]), f32(gm["B"])
        dp = _lib.make_desc(w.batch, w.seq_len, C, F, E, k, r, w.dtype, "fused", flags | _lib.GATE_F32 | _lib.ADAPTERS_F32)
        prep_m = torch.empty(_lib.prepared_bytes(dp), dtype=torch.uint8, device=dev)
        _lib.prepare_adapters(dp, Am, Bmx, prep_m, sh)
        tm = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, w_value=Wv, w_gate=f32(gm["Wg"]), lora_A=Am, lora_B=Bmx,
                               out=torch.empty(N, C, dtype=torch.float32, device=dev), losses=losses,
                               prepared=prep_m, **extra)
        res = {"layer": "fp16 x and base, fp32 gate and adapters, fp32 out (prepared adapters)"}
        for mode in ("fused", "sparse"):
            dm = _lib.make_desc(w.batch, w.seq_len, C, F, E, k, r, w.dtype, mode,
                                flags | _lib.GATE_F32 | _lib.ADAPTERS_F32)
            nm = _lib.workspace_bytes(dm)
            wsm = torch.empty(nm, dtype=torch.uint8, device=dev)
            mms = time_loop(lambda: _lib.call("rwkvmoe_forward", dm, tm, wsm, nm, sh))
            res[mode] = {"ms_per_step": round(mms, 5), "tokens_per_s": round(N / (mms * 1e-3), 1)}
            del wsm
        return res

    # ---- the backward (VJP for x, lora_A, lora_B, router gate), timed the same
    # way as the forward: K back-to-back calls on the stream, inputs resident
    def time_backward():
        lg = torch.empty(N, E, dtype=torch.float32, device=dev)
        ind = torch.empty(N, k, dtype=torch.int32, device=dev)
        fwd_ex = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, w_value=Wv, w_gate=Wg, lora_A=A, lora_B=B, out=out,
                                   losses=losses, logits=lg, inds=ind, **extra)
        _lib.call("rwkvmoe_forward", desc, fwd_ex, ws, nbytes, sh)
        dO = torch.randn(N, C, generator=torch.Generator().manual_seed(7)).to(dev).to(dt)
        dls = torch.tensor([0.01, 0.001], dtype=torch.float32, device=dev)
        grads = {"d_x": torch.empty_like(x), "d_lora_A": torch.empty_like(A), "d_lora_B": torch.empty_like(B),
                 "d_w_gate": torch.empty_like(Wg)}
        bn = _lib.backward_workspace_bytes(desc)
        bws = torch.empty(bn, dtype=torch.uint8, device=dev)

        def bstep():
            _lib.backward(desc, bws, bn, sh, x=x, w_gate=Wg, lora_A=A, lora_B=B, logits=lg, inds=ind, d_out=dO,
                          d_losses=dls, **grads)

        for _ in range(args.warmup):
            bstep()
        torch.cuda.synchronize()
        b0 = torch.cuda.Event(enable_timing=True)
        b1 = torch.cuda.Event(enable_timing=True)
        hold_queue()
        b0.record(stream)
        for _ in range(args.steps):
            bstep()
        b1.record(stream)
        torch.cuda.synchronize()
        bms = b0.elapsed_time(b1) / args.steps
        return {"ms_per_step": round(bms, 5), "tokens_per_s": round(N / (bms * 1e-3), 1),
                "grads": "d_x, d_lora_A, d_lora_B, d_w_gate (d_out and the aux/z cotangents given)"}

    def time_experts():
        """The full-expert layer (MoE_CMix) of the same shape: E ChannelMix
        experts of d_ffn F, random weights, the same x; timed like the
        forward.  Algorithmic FLOPs: the routed rows' key and value products."""
        rng = np.random.default_rng(11)
        xkE = up(rng.uniform(0, 1, (E, C)).astype(np.float32))
        wkE = up((rng.standard_normal((E, F, C)) / np.sqrt(C)).astype(np.float32))
        wvE = up((rng.standard_normal((E, C, F)) / np.sqrt(F)).astype(np.float32))
        dE = _lib.make_desc(w.batch, w.seq_len, C, F, E, k, 1, w.dtype, _lib.MODE_FUSED, flags)
        en = _lib.experts_workspace_bytes(dE)
        ews = torch.empty(en, dtype=torch.uint8, device=dev)
        te = _lib.make_tensors(x=x, x_k=xkE, w_key=wkE, w_value=wvE, w_gate=Wg, out=out, losses=losses, **extra)

        def estep():
            _lib.call("rwkvmoe_experts_forward", dE, te, ews, en, sh)

        for _ in range(args.warmup):
            estep()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        hold_queue()
        e0.record(stream)
        for _ in range(args.steps):
            estep()
        e1.record(stream)
        torch.cuda.synchronize()
        ems = e0.elapsed_time(e1) / args.steps
        flops = 2.0 * N * k * C * F * 2
        res = {"ms_per_step": round(ems, 5), "tokens_per_s": round(N / (ems * 1e-3), 1),
               "gemm_tflops": round(flops / (ems * 1e-3) / 1e12, 1),
               "layer": f"MoE_CMix, {E} experts of d_ffn {F}, top-{k}, random weights"}
        if args.no_backward:
            return res
        # its VJP (rwkvmoe_experts_backward) for every input and parameter,
        # timed the same way; FLOPs: the key product recomputed, u, dk and the
        # two weight gradients over the routed rows
        lg = torch.empty(N, E, dtype=torch.float32, device=dev)
        ind = torch.empty(N, k, dtype=torch.int32, device=dev)
        tf = _lib.make_tensors(x=x, x_k=xkE, w_key=wkE, w_value=wvE, w_gate=Wg, out=out, losses=losses, logits=lg,
                               inds=ind, **extra)
        _lib.call("rwkvmoe_experts_forward", dE, tf, ews, en, sh)
        dO = torch.randn(N, C, generator=torch.Generator().manual_seed(8)).to(dev).to(dt)
        dls = torch.tensor([0.01, 0.001], dtype=torch.float32, device=dev)
        grads = {"d_x": torch.empty_like(x), "d_x_k": torch.empty_like(xkE), "d_w_key": torch.empty_like(wkE),
                 "d_w_value": torch.empty_like(wvE), "d_w_gate": torch.empty_like(Wg)}
        if "x_prev" in extra:
            grads["d_x_prev"] = torch.empty_like(extra["x_prev"])
        bn = _lib.experts_backward_workspace_bytes(dE)
        bws = torch.empty(bn, dtype=torch.uint8, device=dev)

        def bstep():
            _lib.experts_backward(dE, bws, bn, sh, x=x, x_prev=extra.get("x_prev"), x_k=xkE, w_key=wkE, w_value=wvE,
                                  w_gate=Wg, logits=lg, inds=ind, d_out=dO, d_losses=dls, **grads)

        bms = time_loop(bstep)
        bflops = 2.0 * N * k * C * F * 5
        res["backward"] = {"ms_per_step": round(bms, 5), "tokens_per_s": round(N / (bms * 1e-3), 1),
                           "gemm_tflops": round(bflops / (bms * 1e-3) / 1e12, 1),
                           "grads": "d_x, d_x_prev (with a carried state), d_x_k, d_w_key, d_w_value, d_w_gate"}
        return res

    if args.experts_only:
        print(json.dumps({"workload": w.name, "experts": time_experts()}))
        return
    if args.mixed_only:  # the fp16-base / fp32-adapter layer alone (for kernel traces)
        print(json.dumps({"workload": w.name, "mixed_forward": time_mixed()}))
        return
    if args.block_only:  # the Block form alone (for kernel traces)
        print(json.dumps({"workload": w.name, "block_forward": time_block()}))
        return
    if args.backward_only:  # the backward alone (for per-kernel traces of it)
        print(json.dumps({"workload": w.name, "backward": time_backward()}))
        return

    def step():
        _lib.call("rwkvmoe_forward", desc, fwd, ws, nbytes, sh)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    # a spin kernel ahead of the timed region: the host enqueues all K forwards
    # while it runs, so the events time the GPU's pace, not the host's
    hold_queue()
    t0.record(stream)
    for _ in range(args.steps):
        step()
    t1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = t0.elapsed_time(t1) / args.steps
    tokens_per_s = N / (ms * 1e-3)

    # ---- skewed routing: the logit bias and the load it produced
    routing = None
    if w.zipf_s is not None:
        ind = torch.empty(N, k, dtype=torch.int32, device=dev)
        fwd_i = _lib.make_tensors(x=x, x_k=xk, w_key=Wk, w_value=Wv, w_gate=Wg, lora_A=A, lora_B=B, out=out,
                                  losses=losses, inds=ind, **extra)
        _lib.call("rwkvmoe_forward", desc, fwd_i, ws, nbytes, sh)
        torch.cuda.synchronize()
        sel = ind.cpu().numpy()
        load = np.bincount(sel.reshape(-1), minlength=E)
        routing = {"bias": f"beta * ln p_e, p_e ∝ (e+1)^-{w.zipf_s}", "beta": w.bias_beta,
                   "top1_share_expert0": round(float(np.mean(sel[:, 0] == 0)), 4),
                   "in_topk_share_expert0": round(float(np.mean((sel == 0).any(axis=1))), 4),
                   "assignment_share_expert0": round(float(load[0] / sel.size), 4),
                   "max_over_mean_load": round(float(load.max() / load.mean()), 2)}

    # ---- single forwards: warm, and after a 512 MB write that evicts the
    # 256 MB last-level cache and every L2 (inputs and weights then come from
    # HBM); medians of per-forward event pairs on the same stream
    single = None
    if args.single > 0:
        scratch = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.single)]
        res = {}
        for label, flush in (("warm", False), ("flushed", True)):
            hold_queue()
            for i, (a, b) in enumerate(ev):
                if flush:
                    scratch.fill_(i & 0xFF)
                a.record(stream)
                step()
                b.record(stream)
            torch.cuda.synchronize()
            res[label] = sorted(a.elapsed_time(b) for a, b in ev)[len(ev) // 2]
        single = {"forwards": args.single, "warm_median_ms": round(res["warm"], 5),
                  "flushed_median_ms": round(res["flushed"], 5),
                  "flushed_tokens_per_s": round(N / (res["flushed"] * 1e-3), 1),
                  "flush": "512 MB device write before each forward"}
        if not args.no_kernels:  # which kernels pay for the cold caches
            per = {}
            for label, flush in (("warm", False), ("flushed", True)):
                timer = _lib.KernelTimer(stream, args.single)
                hold_queue()
                for i in range(args.single):
                    if flush:
                        scratch.fill_(i & 0xFF)
                    timer.forward(desc, fwd, ws, nbytes)
                per[label] = {nm: round(us, 2) for nm, us in timer.summary()}
                del timer
            single["kernels_us"] = per
        del scratch

    # ---- the forward captured in HIP graphs and replayed back to back (a
    # serving loop's form: no per-kernel launch cost on the host).  A graph
    # launch has a fixed cost of its own (~5-9 us here), so a loop captures
    # several forwards (layers, steps) per graph; both forms are reported.
    graph = None
    if not args.no_graph:
        def graph_ms(per):
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                for _ in range(per):
                    _lib.call("rwkvmoe_forward", desc, fwd, ws, nbytes, torch.cuda.current_stream(dev).cuda_stream)
            for _ in range(max(2, args.warmup // per)):
                gr.replay()
            torch.cuda.synchronize()
            reps = max(2, args.steps // per)
            g0 = torch.cuda.Event(enable_timing=True)
            g1 = torch.cuda.Event(enable_timing=True)
            hold_queue()
            g0.record(stream)
            for _ in range(reps):
                gr.replay()
            g1.record(stream)
            torch.cuda.synchronize()
            del gr
            return g0.elapsed_time(g1) / (reps * per)
        g1ms, g10ms = graph_ms(1), graph_ms(10)
        graph = {"ms_per_step": round(g10ms, 5), "tokens_per_s": round(N / (g10ms * 1e-3), 1),
                 "form": "10 forwards captured in one HIP graph, replayed back to back (per forward)",
                 "one_forward_per_graph": {"ms_per_step": round(g1ms, 5), "tokens_per_s": round(N / (g1ms * 1e-3), 1),
                                           "form": "one forward per graph: each replay pays the graph launch"}}

    # the forward that lays the adapters out itself, and the layout pass alone
    ums = time_loop(lambda: _lib.call("rwkvmoe_forward", desc, fwd_raw, ws, nbytes, sh))
    unprepared = {"ms_per_step": round(ums, 5), "tokens_per_s": round(N / (ums * 1e-3), 1),
                  "form": "rwkvmoe_forward without prepared adapters" + (" or base" if pbase is not None else "")
                          + " (the layout pass in every forward)"}
    pms = time_loop(lambda: _lib.prepare_adapters(desc, A, B, prep, sh))
    backward = None if args.no_backward else time_backward()
    experts = None if args.no_experts else time_experts()
    sparse = time_sparse() if args.mode == "fused" else None
    mixed = time_mixed()
    block = time_block()
    block["over_layer"] = round(block["ms_per_step"] / ms, 4)
    if mixed is not None:
        mixed["fused_over_fp16_layer"] = round(mixed["fused"]["ms_per_step"] / ms, 4)

    # ---- every kernel of the forward, timed on its launch stream -------------
    # the adapter down-projection runs in the router for 16-bit layers with
    # E*r <= 128 and 16-token router workgroups, else in the key GEMM (FUSED)
    # or in the grouped LoRA (SPARSE)
    router_u = w.dtype != "f32" and E * r <= 128 and router_tile_tokens(w, s) == 16
    tables = {}
    if not args.no_kernels:
        for mode in dict.fromkeys([args.mode, "fused", "sparse"]):
            d2, ws2, nb2 = (desc, ws, nbytes) if mode == args.mode else setup(mode)
            for _ in range(args.warmup):
                _lib.call("rwkvmoe_forward", d2, fwd, ws2, nb2, sh)
            per = []
            for pairs in (True, False):
                timer = _lib.KernelTimer(stream, args.steps, pairs=pairs)
                hold_queue()  # the host enqueues every timed forward before the GPU starts them
                for _ in range(args.steps):
                    timer.forward(d2, fwd, ws2, nb2)
                per.append(timer.summary())
                del timer
            # SPARSE takes the router's adapter product where its value launch
            # carries the rank slices (cmix_value_sparse)
            ru = router_u if mode == "fused" else any(name == "cmix_value_sparse" for name, _ in per[0])
            tables[mode] = kernel_table(per[0], per[1], w, kx, s, w.dtype, ru, overhead)
            if mode == "sparse":
                # the dispatch / grouped LoRA / combine form of the same forward
                per = []
                for pairs in (True, False):
                    timer = _lib.KernelTimer(stream, args.steps, pairs=pairs)
                    hold_queue()
                    for _ in range(args.steps):
                        timer.forward(d2, fwd_rows, ws2, nb2)
                    per.append(timer.summary())
                    del timer
                tables["sparse_grouped"] = kernel_table(per[0], per[1], w, kx, s, w.dtype, False, overhead)
        dom = max(tables[args.mode], key=lambda row: row["us"])
        roofline = {"bound": dom["bound"], "achieved": dom["achieved"], "peak": dom["peak"], "unit": dom["unit"],
                    "frac": dom["frac"], "traffic": traffic_for(w.name, dom["kernel"]), "kernel": dom["kernel"],
                    "kernel_us": dom["us"], "kernel_us_marginal": dom["us_marginal"],
                    "event_overhead_us": round(overhead, 3), "algorithmic": dom["algorithmic"],
                    "algorithmic_unit": dom["algorithmic_unit"],
                    "duration": "the kernel's own begin / end timestamps, recorded by its launch "
                                "(rwkvmoe_forward_timed with per-launch event pairs, hipExtLaunchKernel) on the "
                                "launch stream, mean over the timed forwards",
                    "kernels_sum_us": round(sum(r["us"] for r in tables[args.mode]), 3),
                    "kernels_marginal_sum_us": round(sum(r["us_marginal"] for r in tables[args.mode]), 3),
                    "sums": "kernels_sum_us adds each launch's own begin-to-end time; those spans include the "
                            "timestamp writes of the launch's event pair, so in a stream of back-to-back forwards "
                            "they add up to a little more than ms_per_step.  kernels_marginal_sum_us adds what each "
                            "kernel adds to the stream (its interval between events less an empty kernel's) and "
                            "stays below ms_per_step."}
        tr = kernel_trace_for(w.name, dom["kernel"], args.mode)
        if tr is not None:
            amount = dom["algorithmic"] / (tr[0] * 1e-6) / (1e12 if dom["bound"] == "mfma" else 1e9)
            roofline["rocprof"] = {"kernel_us": tr[0], "trace": tr[1], "achieved": round(amount, 2),
                                   "frac": round(amount / dom["peak"], 4),
                                   "live_over_rocprof": round(dom["us"] / tr[0], 4)}
    else:
        roofline = None
    if args.table:
        for mode, rows in tables.items():
            print(f"-- {mode}", file=sys.stderr)
            for row in rows:
                print(f"{row['kernel']:22s} {row['us']:9.3f} us  {row['achieved']:10.1f} {row['unit']:8s} "
                      f"{100 * row['frac']:6.1f}% of {row['bound']}", file=sys.stderr)

    # ---- CPU baseline: the oracle's restatement of the reference algorithm ----
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(w, g, args.cpu_seconds)
        # the same oracles' restatements for the backward and the full-expert
        # layer, on bounded samples beside their GPU timings
        extra_cpu = cpu_others(w, g, min(args.cpu_seconds, 4.0))
        if backward is not None:
            backward["cpu_baseline"] = extra_cpu["backward"]
        if experts is not None:
            experts["cpu_baseline"] = extra_cpu["experts"]
            if "backward" in experts:
                experts["backward"]["cpu_baseline"] = extra_cpu["experts_backward"]

    # ---- the vendor library on the same plain products (no relu², no adapter
    # columns), for comparison with the key / value kernels above
    blas = None
    if args.vs_hipblaslt:
        blas = {}
        for label, (m_, n_, k_) in (("key", (N, F, C)), ("value", (N, C, F))):
            xa = torch.randn(m_, k_, device=dev).to(dt)
            wb = torch.randn(n_, k_, device=dev).to(dt)
            for _ in range(args.warmup):
                torch.matmul(xa, wb.t())
            torch.cuda.synchronize()
            m0 = torch.cuda.Event(enable_timing=True)
            m1 = torch.cuda.Event(enable_timing=True)
            hold_queue()
            m0.record(stream)
            for _ in range(args.steps):
                torch.matmul(xa, wb.t())
            m1.record(stream)
            torch.cuda.synchronize()
            us = m0.elapsed_time(m1) / args.steps * 1e3
            blas[label] = {"shape_mnk": [m_, n_, k_], "us": round(us, 2),
                           "tflops": round(2.0 * m_ * n_ * k_ / us / 1e6, 1)}
            del xa, wb

    rec = {
        "metric": METRIC if w is HEADLINE else f"MoE-ChannelMix tokens/s + %HBM/%MFMA roofline, {w.name}",
        "value": round(tokens_per_s, 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms, 5), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": w.dtype, "data": "synthetic (seeded N(0,1) inputs, "
        "reference-shaped random weights)",
        "config": {"workload": w.name, "tokens": N, "batch": w.batch, "seq_len": w.seq_len, "d_model": C,
                   "d_ffn": F, "n_experts": E, "top_k": k, "lora_rank": r, "mode": args.mode,
                   "parallelism": "single GPU", **({"routing": routing} if routing else {})},
        "roofline": roofline, "cpu_baseline": cpu, "single_forward": single, "graph_replay": graph,
        "hipblaslt_plain_products": blas,
        "forward_unprepared": unprepared, "prepare_adapters_us": round(pms * 1e3, 2),
        "sparse_forward": sparse, "mixed_forward": mixed, "block_forward": block,
        "backward": backward, "experts": experts,
        "wall_s": round(wall, 4),
        "kernels": tables.get(args.mode), "kernels_sparse": tables.get("sparse") if args.mode != "sparse" else None,
        "kernels_sparse_grouped": tables.get("sparse_grouped"),
    }
    print(json.dumps(rec))


def hold_queue(cycles: int = 1_000_000) -> None:
    """Enqueue a short spin kernel of `cycles` GPU clock cycles on the
    current stream, so that the host enqueues the first timed launches while
    the GPU waits: event intervals then measure the GPU's pace, not the
    host's (the host enqueues a headline forward in ~8 us, the GPU runs one in
    ~60 us, so the host stays ahead after that).  The spin is kept short on
    purpose: behind a 100M-cycle spin (tens of ms of one busy wave) the
    headline forward measured 65-71 us per step against 63 us behind a
    1M-cycle spin or none, on the same box in the same process — the clocks
    settle lower over a long nearly idle stretch and take milliseconds to
    come back."""
    import torch
    torch.cuda._sleep(cycles)


def event_overhead_us(stream, n: int = 200) -> float:
    """What an event-bracketed interval adds to the kernel between its
    events: the median interval between HIP events recorded around an empty
    kernel (torch.cuda._sleep(0)), n times back to back on `stream` behind a
    spin kernel (hold_queue), as rwkvmoe_forward_timed records them around
    each kernel of a forward."""
    import torch
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    hold_queue()
    evs[0].record(stream)
    for i in range(n):
        torch.cuda._sleep(0)
        evs[i + 1].record(stream)
    torch.cuda.synchronize()
    iv = sorted(evs[i].elapsed_time(evs[i + 1]) * 1e3 for i in range(n))
    return iv[n // 2]


def kernel_trace_for(workload: str, kernel: str, mode: str = "fused"):
    """The committed rocprofv3 kernel-trace average of `kernel` (bench's
    launch label) in this workload's forward, from
    profiles/kernels_<workload>.json: (avg_us, trace file) or None."""
    name = f"kernels_{workload}.json"
    try:
        t = json.loads((REPO / "profiles" / name).read_text())
    except (OSError, ValueError):
        return None
    entry = t.get(mode, {}).get(kernel)
    if entry is None:
        return None
    return entry["avg_us"], "profiles/" + t.get("trace", name)


def traffic_for(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed counter summary of
    the workload (FETCH_SIZE + WRITE_SIZE, scaled by a copy kernel of known
    size), if any."""
    try:
        t = json.loads((REPO / "profiles" / f"traffic_{workload}.json").read_text())
    except (OSError, ValueError):
        return None
    entry = t.get("kernels", {}).get(kernel)
    return None if entry is None else entry.get("bytes")


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


def cpu_others(w, g, budget_s):
    """Oracle timings for the backward (float64 VJP restatement) and the
    full-expert layer (the reference's dense expert loop, fp32 products), each
    on one 64-token sequence repeated within ``budget_s`` seconds."""
    import numpy as np

    from oracle import moe_backward as MB
    from oracle import moe_oracle as O
    T = 64
    C, F, E, k = w.d_model, w.d_ffn, w.n_experts, w.top_k
    x = g["x"].reshape(-1, C)[:T]
    rng = np.random.default_rng(3)
    dO = O.round_to(rng.standard_normal((T, C)), w.dtype)
    pe = {"x_k": O.round_to(rng.uniform(0, 1, (E, C)), w.dtype),
          "Wk": O.round_to(rng.standard_normal((E, F, C)) / np.sqrt(C), w.dtype),
          "Wv": O.round_to(rng.standard_normal((E, C, F)) / np.sqrt(F), w.dtype), "Wg": g["Wg"]}

    def timed(fn):
        fn()
        times = []
        t_end = time.perf_counter() + budget_s
        while time.perf_counter() < t_end or len(times) < 2:
            t = time.perf_counter()
            fn()
            times.append(time.perf_counter() - t)
        return float(np.median(times)), len(times)

    bmed, bn = timed(lambda: MB.moe_backward(x, g["Wg"], g["A"], g["B"], k, w.dtype, dO, 0.01, 0.001))
    emed, en = timed(lambda: O.experts_forward(x[None], pe, k, w.dtype, mm_dtype=np.float32))
    xbmed, xbn = timed(lambda: MB.experts_backward(x[None], pe, k, w.dtype, dO[None], 0.01, 0.001))
    return {"experts_backward": {"value": round(T / xbmed, 1), "unit": "tokens/s", "kind": "port",
                                 "sample": f"oracle experts_backward (NumPy float64 VJP, the dense loop over all "
                                           f"{E} experts) on {T} tokens, median of {xbn} runs"},
            "backward": {"value": round(T / bmed, 1), "unit": "tokens/s", "kind": "port",
                         "sample": f"oracle moe_backward (NumPy float64 VJP) on {T} tokens, median of {bn} runs"},
            "experts": {"value": round(T / emed, 1), "unit": "tokens/s", "kind": "port",
                        "sample": f"oracle experts_forward (NumPy, fp32 products, the dense loop over all {E} "
                                  f"experts) on {T} tokens, median of {en} runs"}}


if __name__ == "__main__":
    main()
