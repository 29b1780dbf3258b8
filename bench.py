#!/usr/bin/env python3
"""Benchmark of the MI355X Roformer hot path.

Workload (one step = one 8 s chunk through the transformer stack):
  BSRoformer transformer stack, depth 12 (12 time + 12 frequency layers),
  dim 512, 8 heads x 64, FF 512->2048->512 with GELU, RMSNorm, RoPE and
  sigmoid gates; activation [1 chunk, 801 frames, 62 bands, 512], fp16
  weights/activations, fp32 accumulation and fp32 residual stream.
  Weights ~ N(0, 0.02) (gammas 1 + N(0, 0.02)), x ~ N(0, 1), seed 0,
  generated on the device (synthetic: no checkpoint is available).

Prints ONE JSON line:
  value          ms per 8 s chunk (lower is better), inputs resident in HBM
  gemm_tflops    the stack's MFMA GEMMs replayed alone (same shapes, same
                 epilogues, same stream) -> TFLOP/s and fraction of peak
  roofline       dominant kernel = gemm_f16_kernel on the FF1 shape
                 (M=49662, K=512, N=2048, bias+GELU, fp16 out), HIP-event
                 timed over the launches of its own timed loop
  cpu_baseline   the fp32 CPU oracle on a bounded sample (one depth of the
                 stack = 1/12 of the chunk), extrapolated to ms per chunk
  parity         GPU vs oracle on that same one-depth sample
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "cuda-msst-infer_amd")

METRIC = "ms per 8s chunk + GEMM TFLOP/s (% MFMA peak), BSRoformer fp16, 1×MI355X"
PEAK_F16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA, published
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E, published

# BSRoformer config: [62 bands, 801 frames] per 8 s chunk (44.1 kHz, hop 441).
FRAMES, BANDS, DIM, HEADS, DH, FF, DEPTH = 801, 62, 512, 8, 64, 2048, 12


def load_msst():
    if "msst_amd" in sys.modules:
        return sys.modules["msst_amd"]
    spec = importlib.util.spec_from_file_location(
        "msst_amd", os.path.join(PKG_DIR, "__init__.py"), submodule_search_locations=[PKG_DIR])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["msst_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


def gemm_flops_per_token_layer():
    hd = HEADS * DH
    # QKV, out-proj, FF1, FF2 (the 8-wide gate projection runs inside RMSNorm)
    return 2 * (DIM * 3 * hd + hd * DIM + DIM * FF + FF * DIM)


def attn_flops_chunk(batch):
    # QK^T + PV: 4 * N^2 * D per (sequence, head)
    t = batch * BANDS * HEADS * 4 * FRAMES ** 2 * DH
    f = batch * FRAMES * HEADS * 4 * BANDS ** 2 * DH
    return DEPTH * (t + f)


def make_weights(torch, seed, dtype):
    g = torch.Generator(device="cuda").manual_seed(seed)
    hd = HEADS * DH

    def n(*s, dt=dtype):
        return (torch.randn(*s, device="cuda", generator=g) * 0.02).to(dt)

    def gm():
        return 1.0 + torch.randn(DIM, device="cuda", generator=g) * 0.02

    layers = []
    for _ in range(2 * DEPTH):
        layers.append(dict(attn_gamma=gm(), w_qkv=n(3 * hd, DIM), w_gate=n(HEADS, DIM),
                           b_gate=n(HEADS, dt=torch.float32), w_out=n(DIM, hd), ff_gamma=gm(),
                           w_ff1=n(FF, DIM), b_ff1=n(FF, dt=torch.float32), w_ff2=n(DIM, FF),
                           b_ff2=n(DIM, dt=torch.float32)))
    return layers, gm()


def time_events(torch, fn, steps):
    s = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(s)
    for _ in range(steps):
        fn()
    stop.record(s)
    torch.cuda.synchronize()
    return start.elapsed_time(stop)


def gemm_replay(msst, torch, layers, batch):
    """The stack's MFMA GEMM launches for one chunk, same shapes/epilogues."""
    M = batch * FRAMES * BANDS
    hd = HEADS * DH
    xn = torch.randn(M, DIM, device="cuda").half()
    qkv = torch.empty(M, 3 * hd, device="cuda", dtype=torch.float16)
    merged = torch.randn(M, hd, device="cuda").half()
    hidden = torch.empty(M, FF, device="cuda", dtype=torch.float16)
    res = torch.randn(M, DIM, device="cuda")

    def run():
        for w in layers:
            msst.linear(xn, w["w_qkv"], out=qkv)
            msst.linear(merged, w["w_out"], residual=res, out=res)
            msst.linear(xn, w["w_ff1"], w["b_ff1"], "gelu", out=hidden)
            msst.linear(hidden, w["w_ff2"], w["b_ff2"], residual=res, out=res)
    return run


def cpu_baseline_and_parity(msst, torch, args):
    """Oracle on one depth (time + frequency transformer) of the stack at
    full size; the GPU runs the same depth for the parity figure."""
    import numpy as np
    sys.path.insert(0, ROOT)
    from oracle import oracle as O
    threads = O.num_threads()
    rng = np.random.default_rng(0)
    hd = HEADS * DH

    def n(*s):
        return (rng.standard_normal(s) * 0.02).astype(np.float16).astype(np.float32)

    def gm():
        return (1 + rng.standard_normal(DIM) * 0.02).astype(np.float32)

    lw = []
    for _ in range(2):
        lw.append(dict(attn_gamma=gm(), w_qkv=n(3 * hd, DIM), w_gate=n(HEADS, DIM),
                       b_gate=n(HEADS), w_out=n(DIM, hd), ff_gamma=gm(), w_ff1=n(FF, DIM),
                       b_ff1=n(FF), w_ff2=n(DIM, FF), b_ff2=n(DIM)))
    x = rng.standard_normal((1, FRAMES, BANDS, DIM)).astype(np.float32)
    t0 = time.perf_counter()
    ref = O.roformer_stack(x, [O.LayerWeights(**w) for w in lw], HEADS, DH, None)
    cpu_s = time.perf_counter() - t0

    mats = ("w_qkv", "w_gate", "w_out", "w_ff1", "w_ff2")
    dl = [{k: (torch.from_numpy(v).cuda().half() if k in mats else torch.from_numpy(v).cuda())
           for k, v in w.items()} for w in lw]
    st = msst.RoformerStack(dl, None, 1, FRAMES, BANDS, DIM, HEADS, DH, FF, msst.F16)
    xd = torch.from_numpy(x).cuda()
    st(xd)
    torch.cuda.synchronize()
    y = xd.cpu().numpy().astype(np.float64)
    err = float(np.max(np.abs(y - ref)) / np.max(np.abs(ref)))
    cpu = {"value": round(cpu_s * 1e3 * DEPTH, 1), "unit": "ms/chunk", "cores": threads,
           "kind": "port",
           "sample": "fp32 C oracle, one depth (time + frequency transformer) of the "
                     "12-depth stack at full size [801 frames x 62 bands x 512], "
                     f"measured {cpu_s:.2f} s, extrapolated x{DEPTH}"}
    parity = {"max_rel_err": err, "tolerance": 2e-2, "metric": "max|y-r|/max|r|",
              "sample": "same one-depth stack, fp16 HIP path vs fp32 oracle"}
    return cpu, parity


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=1, help="chunks per step (config 5 uses 4)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(chunk-level data parallelism across GPUs is described in DESIGN.md).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    msst = load_msst()
    msst.lib()
    torch.manual_seed(0)
    B = args.batch
    layers, final_gamma = make_weights(torch, 0, torch.float16)
    st = msst.RoformerStack(layers, final_gamma, B, FRAMES, BANDS, DIM, HEADS, DH, FF, msst.F16)
    x = torch.randn(B, FRAMES, BANDS, DIM, device="cuda",
                    generator=torch.Generator(device="cuda").manual_seed(1))

    for _ in range(args.warmup):
        st(x)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_ms = time_events(torch, lambda: st(x), args.steps)
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = ev_ms / args.steps
    ms_per_chunk = ms_per_step / B
    assert torch.isfinite(x).all().item(), "non-finite stack output"

    # GEMM replay: the stack's GEMM launches alone.
    run = gemm_replay(msst, torch, layers, B)
    run()
    reps = max(2, min(5, args.steps))
    gemm_ms = time_events(torch, run, reps) / reps
    M = B * FRAMES * BANDS
    gemm_flops = gemm_flops_per_token_layer() * M * 2 * DEPTH
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12

    # Dominant kernel: FF1 GEMM (bias + GELU, fp16 out).
    xn = torch.randn(M, DIM, device="cuda").half()
    hid = torch.empty(M, FF, device="cuda", dtype=torch.float16)
    w1, b1 = layers[0]["w_ff1"], layers[0]["b_ff1"]
    msst.linear(xn, w1, b1, "gelu", out=hid)
    nl = 50
    ff1_ms = time_events(torch, lambda: msst.linear(xn, w1, b1, "gelu", out=hid), nl) / nl
    ff1_flops = 2.0 * M * DIM * FF
    ff1_tflops = ff1_flops / (ff1_ms * 1e-3) / 1e12
    ff1_bytes = 2 * M * DIM + 2 * FF * DIM + 4 * FF + 2 * M * FF

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "gemm_ff1_traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": round(ms_per_chunk, 3),
        "unit": "ms/chunk",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) input, generated on device)",
        "config": {
            "workload": "BSRoformer transformer stack, one 8 s chunk: depth 12 (time + "
                        "frequency layer each), dim 512, 8 heads x 64, FF 2048 GELU, RMSNorm, "
                        "RoPE, sigmoid gates; time layers on [62, 801, 512], frequency layers "
                        "on [801, 62, 512]; fp16 weights/activations, fp32 accumulation and "
                        "residual",
            "chunks_per_step": B, "frames": FRAMES, "bands": BANDS, "dim": DIM, "depth": DEPTH,
        },
        "wall_ms_timed_region": round(wall_ms, 2),
        "gemm_ms_per_chunk": round(gemm_ms / B, 3),
        "gemm_tflops": round(gemm_tflops, 1),
        "gemm_frac_of_peak": round(gemm_tflops / PEAK_F16_TFLOPS, 4),
        "stack_tflops": round((gemm_flops + attn_flops_chunk(B)) / (ms_per_step * 1e-3) / 1e12, 1),
        "roofline": {
            "kernel": "gemm_f16_kernel<256,256> FF1 M=49662 K=512 N=2048 bias+GELU fp16 out"
                      if B == 1 else f"gemm_f16_kernel<256,256> FF1 M={M} K=512 N=2048",
            "bound": "mfma",
            "achieved": round(ff1_tflops, 1),
            "peak": PEAK_F16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(ff1_tflops / PEAK_F16_TFLOPS, 4),
            "traffic": traffic,
            "algorithmic_bytes": ff1_bytes,
            "launch_us": round(ff1_ms * 1e3, 2),
        },
    }
    if not args.no_cpu:
        cpu, parity = cpu_baseline_and_parity(msst, torch, args)
        out["cpu_baseline"] = cpu
        out["parity"] = parity
    print(json.dumps(out))


if __name__ == "__main__":
    main()
