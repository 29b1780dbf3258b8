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
  roofline       dominant kernel = gemm_pp_kernel (256x256 ping-pong tiles,
                 8 waves, bias+GELU epilogue, nt stores) on the FF1 shape
                 (M=49662, K=512, N=2048, bias+GELU, fp16 out), HIP-event
                 timed over 50 launches on the stream it runs on; traffic =
                 HBM bytes per launch from rocprofv3 FETCH_SIZE/WRITE_SIZE
                 (profiles/gemm_ff1_traffic.json), copy-kernel calibrated
  kernels        every kernel of one transformer, timed alone (us/launch),
                 with TFLOP/s (MFMA-bound) or GB/s (HBM-bound)
  cpu_baseline   the fp32 CPU oracle on one whole chunk (about 10 s of CPU
                 work on 16 threads)
  parity         GPU vs oracle on that same chunk (same weights and input)
  pcie_inclusive_ms_per_chunk
                 the same step with the chunk handed over in pinned host
                 memory (H2D copy + stack + D2H copy); never `value`
  config5_batch4 four chunks per step (M = 198648): ms per chunk = step / 4
  config1_fp32_layer
                 one MelBandRoformer time layer in fp32 on [60, 801, 384] and
                 its fp32 kernels against the fp32 matrix peak
  config2_gemm_sweep
                 every (M, K, N, epilogue, dtype) of the GEMM sweep alone:
                 TFLOP/s and fraction of the matrix peak, or GB/s and the
                 fraction of HBM peak for the N = 8 gate projection
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
PEAK_F32_TFLOPS = 157.3    # MI355X fp32 matrix, published
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


def make_weights(torch, seed, dtype, dim=DIM, ff=FF, depth=DEPTH, per_layer_norm=False):
    """Seeded weights of a 2 * depth transformer stack; per_layer_norm: the
    MelBandRoformer form (a norm closing every transformer, no final norm)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    hd = HEADS * DH

    def n(*s, dt=dtype):
        return (torch.randn(*s, device="cuda", generator=g) * 0.02).to(dt)

    def gm():
        return 1.0 + torch.randn(dim, device="cuda", generator=g) * 0.02

    layers = []
    for _ in range(2 * depth):
        lw = dict(attn_gamma=gm(), w_qkv=n(3 * hd, dim), w_gate=n(HEADS, dim),
                  b_gate=n(HEADS, dt=torch.float32), w_out=n(dim, hd), ff_gamma=gm(),
                  w_ff1=n(ff, dim), b_ff1=n(ff, dt=torch.float32), w_ff2=n(dim, ff),
                  b_ff2=n(dim, dt=torch.float32))
        if per_layer_norm:
            lw["final_gamma"] = gm()
        layers.append(lw)
    return layers, (None if per_layer_norm else gm())


def mbr_stack_time(msst, torch, steps):
    """The MelBandRoformer stack of the same 8 s chunk (depth 6, dim 384,
    FF 1536, 60 bands, a norm after every transformer), timed like the
    headline workload; reported beside it, not as the metric."""
    bands, dim, ff, depth = 60, 384, 1536, 6
    layers, _ = make_weights(torch, 2, torch.float16, dim, ff, depth, per_layer_norm=True)
    st = msst.RoformerStack(layers, None, 1, FRAMES, bands, dim, HEADS, DH, ff, msst.F16)
    x = torch.randn(1, FRAMES, bands, dim, device="cuda",
                    generator=torch.Generator(device="cuda").manual_seed(3))
    for _ in range(2):
        st(x)
    ms = time_events(torch, lambda: st(x), steps) / steps
    assert torch.isfinite(x).all().item(), "non-finite MelBandRoformer stack output"
    M = FRAMES * bands
    hd = HEADS * DH
    flops = 2 * depth * M * 2 * (dim * 3 * hd + hd * dim + dim * ff + ff * dim)
    return {"ms_per_chunk": round(ms, 3), "gemm_flops_per_chunk": flops,
            "config": "MelBandRoformer stack, one 8 s chunk: depth 6, dim 384, 8 heads x 64, "
                      "FF 1536 GELU, time layers on [60, 801, 384], frequency layers on "
                      "[801, 60, 384], a norm after every transformer; fp16 weights"}


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
    tcos, tsin = msst.rope_table_device(FRAMES, DH)
    fcos, fsin = msst.rope_table_device(BANDS, DH)

    def run():
        for i, w in enumerate(layers):
            # QKV with the RoPE epilogue, time / frequency positions as in the stack.
            if i % 2 == 0:
                msst.linear_rope(xn, w["w_qkv"], tcos, tsin, 2 * hd, DH, 1, FRAMES, out=qkv)
            else:
                msst.linear_rope(xn, w["w_qkv"], fcos, fsin, 2 * hd, DH, FRAMES, BANDS, out=qkv)
            msst.linear(merged, w["w_out"], residual=res, out=res)
            msst.linear(xn, w["w_ff1"], w["b_ff1"], "gelu", out=hidden)
            msst.linear(hidden, w["w_ff2"], w["b_ff2"], residual=res, out=res)
    return run


def host_cpu_model():
    """The host CPU's model name (lscpu 'Model name', else /proc/cpuinfo)."""
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def batch4_stack(msst, torch, layers, final_gamma, steps):
    """Four overlapped 8 s chunks in one step (time layers on
    [248, 801, 512], frequency layers on [3204, 62, 512], M = 198648);
    ms per chunk = step time / 4, and the GEMM replay at the same M."""
    B = 4
    st = msst.RoformerStack(layers, final_gamma, B, FRAMES, BANDS, DIM, HEADS, DH, FF, msst.F16)
    x = torch.randn(B, FRAMES, BANDS, DIM, device="cuda",
                    generator=torch.Generator(device="cuda").manual_seed(4))
    for _ in range(2):
        st(x)
    ms = time_events(torch, lambda: st(x), steps) / steps
    assert torch.isfinite(x).all().item(), "non-finite batched stack output"
    run = gemm_replay(msst, torch, layers, B)
    run()
    gms = time_events(torch, run, 2) / 2
    M = B * FRAMES * BANDS
    gflops = gemm_flops_per_token_layer() * M * 2 * DEPTH
    tf = gflops / (gms * 1e-3) / 1e12
    return {"ms_per_step": round(ms, 3), "ms_per_chunk": round(ms / B, 3),
            "gemm_ms_per_chunk": round(gms / B, 3), "gemm_tflops": round(tf, 1),
            "gemm_frac_of_peak": round(tf / PEAK_F16_TFLOPS, 4),
            "stack_tflops": round((gflops + attn_flops_chunk(B)) / (ms * 1e-3) / 1e12, 1),
            "config": "BSRoformer stack, 4 chunks per step (time layers on [248, 801, 512], "
                      "frequency layers on [3204, 62, 512], M = 198648), depth 12, fp16"}


def gemm_sweep(msst, torch):
    """Every (M, K, N, epilogue, dtype) of the GEMM sweep, each GEMM
    HIP-event timed alone (10 launches after one warm-up).  fp16: x, W fp16,
    fp32 accumulation, fp16 out; fp32: x, W, out fp32 (true fp32 MFMA).
    Bias ~ N(0, 0.02), A ~ N(0, 1), W ~ N(0, 0.02).  MFMA-bound shapes
    report TFLOP/s and the fraction of the dtype's matrix peak; N = 8 (the
    gate projection) is HBM-bound and reports GB/s of its algorithmic bytes
    (A read once, W, bias, out written once) and the fraction of HBM peak."""
    gen = torch.Generator(device="cuda").manual_seed(9)
    out = []
    shapes = [(384, 1536), (1536, 384), (512, 1536), (512, 2048), (2048, 512), (384, 8), (512, 8)]
    for M in (48060, 49662, 198648):
        for K, N in shapes:
            a32 = torch.randn(M, K, device="cuda", generator=gen)
            w32 = torch.randn(N, K, device="cuda", generator=gen) * 0.02
            b = torch.randn(N, device="cuda", generator=gen) * 0.02
            for dt in ("f16", "f32"):
                tdt = torch.float16 if dt == "f16" else torch.float32
                a, w = a32.to(tdt), w32.to(tdt)
                o = torch.empty(M, N, device="cuda", dtype=tdt)
                for epi in ("none", "gelu", "sigmoid"):
                    fn = lambda: msst.linear(a, w, b, epi, out=o)
                    fn()
                    us = time_events(torch, fn, 10) / 10 * 1e3
                    flops = 2.0 * M * K * N
                    eb = 2 if dt == "f16" else 4
                    nbytes = eb * (M * K + N * K + M * N) + 4 * N
                    e = {"M": M, "K": K, "N": N, "epilogue": epi, "dtype": dt,
                         "us": round(us, 2), "tflops": round(flops / (us * 1e-6) / 1e12, 1)}
                    if N <= 16:
                        gbs = nbytes / (us * 1e-6) / 1e9
                        e.update({"bound": "hbm", "gbs": round(gbs, 1),
                                  "frac_hbm": round(gbs / PEAK_HBM_GBS, 4)})
                    else:
                        peak = PEAK_F16_TFLOPS if dt == "f16" else PEAK_F32_TFLOPS
                        e.update({"bound": "mfma", "frac_mfma": round(e["tflops"] / peak, 4)})
                    out.append(e)
            del a32, w32, a, w, o
    torch.cuda.empty_cache()
    return out


def fp32_mbr_time_layer(msst, torch):
    """On the GPU: one MelBandRoformer time layer in fp32 on
    x [60, 801, 384] (fp32 weights ~ N(0, 0.02), true fp32 MFMA), the whole
    layer HIP-event timed, and each fp32 kernel alone against the fp32
    matrix peak (the attention's QK^T + PV flops as MFMA work)."""
    F, T, dim, heads, ff = 60, 801, 384, 8, 1536
    hd = heads * DH
    g = torch.Generator(device="cuda").manual_seed(11)

    def n(*sh):
        return torch.randn(*sh, device="cuda", generator=g) * 0.02

    def gm():
        return 1.0 + torch.randn(dim, device="cuda", generator=g) * 0.02

    lw = dict(attn_gamma=gm(), w_qkv=n(3 * hd, dim), w_gate=n(heads, dim), b_gate=n(heads),
              w_out=n(dim, hd), ff_gamma=gm(), w_ff1=n(ff, dim), b_ff1=n(ff), w_ff2=n(dim, ff),
              b_ff2=n(dim))
    st = msst.RoformerStack([lw, lw], None, 1, T, F, dim, heads, DH, ff, msst.F32)
    x = torch.randn(F, T, dim, device="cuda", generator=g)
    st.transformer(x, 0, 0)
    layer_ms = time_events(torch, lambda: st.transformer(x, 0, 0), 5) / 5
    M = F * T
    gemm_flops = 2.0 * M * (dim * 3 * hd + hd * dim + dim * ff + ff * dim)
    att_flops = 4.0 * F * heads * T * T * DH
    xn = torch.randn(M, dim, device="cuda", generator=g)
    merged = torch.randn(M, hd, device="cuda", generator=g)
    qkv = torch.empty(M, 3 * hd, device="cuda")
    hid = torch.empty(M, ff, device="cuda")
    res = torch.randn(M, dim, device="cuda", generator=g)
    q, k, v = (torch.randn(F, heads, T, DH, device="cuda", generator=g) for _ in range(3))
    kern = {}
    for name, fn, flops in (
            ("gemm_qkv", lambda: msst.linear(xn, lw["w_qkv"], out=qkv), 2.0 * M * dim * 3 * hd),
            ("gemm_out_residual", lambda: msst.linear(merged, lw["w_out"], residual=res, out=res),
             2.0 * M * hd * dim),
            ("gemm_ff1_gelu", lambda: msst.linear(xn, lw["w_ff1"], lw["b_ff1"], "gelu", out=hid),
             2.0 * M * dim * ff),
            ("gemm_ff2_residual", lambda: msst.linear(hid, lw["w_ff2"], lw["b_ff2"],
                                                      residual=res, out=res), 2.0 * M * ff * dim),
            ("attention", lambda: msst.attention(q, k, v), att_flops)):
        fn()
        us = time_events(torch, fn, 10) / 10 * 1e3
        tf = flops / (us * 1e-6) / 1e12
        kern[name] = {"us": round(us, 1), "tflops": round(tf, 1),
                      "frac_fp32_peak": round(tf / PEAK_F32_TFLOPS, 4)}
    gemm_us = sum(kern[k]["us"] for k in kern if k.startswith("gemm"))
    return {"layer_ms": round(layer_ms, 3),
            "layer_tflops": round((gemm_flops + att_flops) / (layer_ms * 1e-3) / 1e12, 1),
            "gemm_tflops": round(gemm_flops / (gemm_us * 1e-6) / 1e12, 1),
            "gemm_frac_fp32_peak": round(gemm_flops / (gemm_us * 1e-6) / 1e12 / PEAK_F32_TFLOPS, 4),
            "kernels": kern,
            "config": "MelBandRoformer time layer, fp32 weights and activations, x [60, 801, 384], "
                      "8 heads x 64, FF 1536 GELU; peak: fp32 matrix 157.3 TFLOP/s"}


def cpu_baseline_and_parity(msst, torch, args):
    """Oracle on the whole workload (one 8 s chunk through the 12-depth
    stack, BSRoformer final norm) with its own seeded weights — about 10 s of
    CPU work on 16 host threads; the GPU runs the same stack on the same
    weights and input for the parity figure."""
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
    for _ in range(2 * DEPTH):
        lw.append(dict(attn_gamma=gm(), w_qkv=n(3 * hd, DIM), w_gate=n(HEADS, DIM),
                       b_gate=n(HEADS), w_out=n(DIM, hd), ff_gamma=gm(), w_ff1=n(FF, DIM),
                       b_ff1=n(FF), w_ff2=n(DIM, FF), b_ff2=n(DIM)))
    fg = gm()
    x = rng.standard_normal((1, FRAMES, BANDS, DIM)).astype(np.float32)
    t0 = time.perf_counter()
    ref = O.roformer_stack(x, [O.LayerWeights(**w) for w in lw], HEADS, DH, fg)
    cpu_s = time.perf_counter() - t0

    mats = ("w_qkv", "w_gate", "w_out", "w_ff1", "w_ff2")
    dl = [{k: (torch.from_numpy(v).cuda().half() if k in mats else torch.from_numpy(v).cuda())
           for k, v in w.items()} for w in lw]
    st = msst.RoformerStack(dl, torch.from_numpy(fg).cuda(), 1, FRAMES, BANDS, DIM, HEADS, DH,
                            FF, msst.F16)
    xd = torch.from_numpy(x).cuda()
    st(xd)
    torch.cuda.synchronize()
    y = xd.cpu().numpy().astype(np.float64)
    err = float(np.max(np.abs(y - ref)) / np.max(np.abs(ref)))
    cpu = {"value": round(cpu_s * 1e3, 1), "unit": "ms/chunk", "cores": threads,
           "cpu_model": host_cpu_model(), "kind": "port",
           "sample": "fp32 C oracle (OpenMP), one whole 8 s chunk: the 12-depth stack with "
                     "final norm at full size [801 frames x 62 bands x 512], "
                     f"measured {cpu_s:.2f} s"}
    parity = {"max_rel_err": err, "tolerance": 2e-2, "metric": "max|y-r|/max|r|",
              "sample": "the same 12-depth chunk, same weights and input: fp16 HIP path vs "
                        "fp32 oracle"}
    return cpu, parity


def ff1_inputs(torch, layers, M):
    xn = torch.randn(M, DIM, device="cuda",
                     generator=torch.Generator(device="cuda").manual_seed(2)).half()
    hid = torch.empty(M, FF, device="cuda", dtype=torch.float16)
    return xn, hid, layers[0]["w_ff1"], layers[0]["b_ff1"]


def pmc_sample(msst, torch, B, which):
    """Launch sequence for the counter passes, synchronised, nothing timed.

    which == "ff1": a plain copy kernel of known size (256 MiB read + 256 MiB
    written, fp32 negation), then the FF1 GEMM, three launches each (the
    traffic calibration).  which == "kernels": the copy, then every kernel of
    one transformer in stack order, three launches each (kernel_table's
    launches; the counter tables split the dispatches in that order)."""
    layers, _ = make_weights(torch, 0, torch.float16)
    src = torch.randn(64 << 20, device="cuda")
    dst = torch.empty_like(src)
    if which == "ff1":
        xn, hid, w1, b1 = ff1_inputs(torch, layers, B * FRAMES * BANDS)
        ents = [("gemm_ff1_gelu", lambda: msst.linear(xn, w1, b1, "gelu", out=hid))]
    else:
        ents = [(name, fn) for name, fn, _, _ in kernel_ops(msst, torch, layers, B)]
    torch.cuda.synchronize()
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    for _, fn in ents:
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
    print(json.dumps({"pmc_sample": "copy 268435456 B read + 268435456 B written x3; then x3 "
                                    "each: " + ", ".join(n for n, _ in ents)}))


def kernel_ops(msst, torch, layers, B):
    """Every kernel of one transformer as (name, launch, flops, bytes), on
    seeded inputs of the stack's shapes."""
    M = B * FRAMES * BANDS
    hd = HEADS * DH
    w = layers[0]
    gen = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(M, DIM, device="cuda", generator=gen)
    xn = torch.empty(M, DIM, device="cuda", dtype=torch.float16)
    gates = torch.empty(M, HEADS, device="cuda")
    qkv = torch.empty(M, 3 * hd, device="cuda", dtype=torch.float16)
    merged = torch.empty(M, hd, device="cuda", dtype=torch.float16)
    hidden = torch.empty(M, FF, device="cuda", dtype=torch.float16)
    res = torch.randn(M, DIM, device="cuda", generator=gen)
    tcos, tsin = msst.rope_table_device(FRAMES, DH)
    fcos, fsin = msst.rope_table_device(BANDS, DH)
    scale = math.sqrt(DIM)
    # Token order [B, FRAMES, BANDS] as in the stack: time sequences are
    # strided by BANDS tokens, frequency sequences contiguous.
    time_l = msst.seq_layout(B, BANDS, FRAMES, FRAMES * BANDS, 1, BANDS)
    freq_l = msst.seq_layout(B * FRAMES, 1, BANDS, BANDS, 0, 1)
    # (name, fn, flops, bytes) — bytes count each tensor read/written once.
    ents = [
        ("rms_norm_gate", lambda: msst.rms_norm_gate(x, w["attn_gamma"], scale, w["w_gate"],
                                                     w["b_gate"], out=xn, gates=gates),
         0, M * DIM * (4 + 2) + M * HEADS * 4),
        ("gemm_qkv_rope", lambda: msst.linear_rope(xn, w["w_qkv"], tcos, tsin, 2 * hd, DH, BANDS,
                                                   FRAMES, out=qkv),
         2.0 * M * DIM * 3 * hd, 2 * M * DIM + 2 * 3 * hd * DIM + 2 * M * 3 * hd),
        ("attention_time", lambda: msst.gated_rope_attention(qkv, time_l, HEADS, None, None,
                                                             gates, out=merged),
         4.0 * B * BANDS * HEADS * FRAMES ** 2 * DH, 2 * M * 3 * hd + 2 * M * hd + 4 * M * HEADS),
        ("attention_freq", lambda: msst.gated_rope_attention(qkv, freq_l, HEADS, None, None,
                                                             gates, out=merged),
         4.0 * B * FRAMES * HEADS * BANDS ** 2 * DH, 2 * M * 3 * hd + 2 * M * hd + 4 * M * HEADS),
        ("gemm_out_residual", lambda: msst.linear(merged, w["w_out"], residual=res, out=res),
         2.0 * M * hd * DIM, 2 * M * hd + 2 * DIM * hd + 8 * M * DIM),
        ("rms_norm", lambda: msst.rms_norm(res, w["ff_gamma"], scale, out=xn),
         0, M * DIM * (4 + 2)),
        ("gemm_ff1_gelu", lambda: msst.linear(xn, w["w_ff1"], w["b_ff1"], "gelu", out=hidden),
         2.0 * M * DIM * FF, 2 * M * DIM + 2 * FF * DIM + 2 * M * FF),
        ("gemm_ff2_residual", lambda: msst.linear(hidden, w["w_ff2"], w["b_ff2"], residual=res,
                                                  out=res),
         2.0 * M * FF * DIM, 2 * M * FF + 2 * DIM * FF + 8 * M * DIM),
    ]
    return ents


def kernel_table(msst, torch, layers, B):
    """Each kernel of one transformer alone, HIP-event timed on the stream it
    runs on (50 launches after one warm-up)."""
    ents = kernel_ops(msst, torch, layers, B)
    table = {}
    for name, fn, flops, nbytes in ents:
        fn()
        us = time_events(torch, fn, 50) / 50 * 1e3
        e = {"us": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1),
             "frac_hbm": round(nbytes / (us * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)}
        if flops:
            tf = flops / (us * 1e-6) / 1e12
            e.update({"tflops": round(tf, 1), "frac_mfma": round(tf / PEAK_F16_TFLOPS, 4)})
        table[name] = e
    return table


# BSRoformer's band layout: 62 bands over 1025 STFT bins, stereo (2 * freqs
# * 2 channels features per band); mask-estimator MLP of 2 linears, hidden
# 4 * dim (mlp_expansion_factor 4).
BSR_FREQS = [2] * 24 + [4] * 12 + [12] * 8 + [24] * 8 + [48] * 8 + [128, 129]


def band_table(msst, torch, B):
    """Band gather, band split, one stem's mask estimator and the mask merge
    on one chunk's frames (rows = B * 801), HIP-event timed, 50 launches
    after one warm-up."""
    dims = [4 * f for f in BSR_FREQS]
    rows, nb, hid, ftot = B * FRAMES, len(dims), 4 * DIM, sum(dims)
    gen = torch.Generator(device="cuda").manual_seed(5)

    def n(*s, sd=0.02, dt=torch.float16):
        return (torch.randn(*s, device="cuda", generator=gen) * sd).to(dt)

    split = ([1.0 + n(d, dt=torch.float32) for d in dims], [n(DIM, d) for d in dims],
             [n(DIM, dt=torch.float32) for d in dims])
    mask = ([[n(hid, DIM), n(2 * d, hid)] for d in dims],
            [[n(hid, dt=torch.float32), n(2 * d, dt=torch.float32)] for d in dims])
    plan = msst.BandPlan(dims, DIM, split=split, mask=mask, channels=2, stft_bins=1025)
    stft = torch.randn(2 * B, 1025, FRAMES, 2, device="cuda", generator=gen)
    x = plan.band_gather(stft, B).reshape(rows, ftot)
    feats = plan.band_split(x)
    m = plan.mask_estimator(feats)
    masks = m.reshape(1, B, FRAMES, ftot)
    # 8 s of stereo audio at 44.1 kHz -> 801 frames (n_fft 2048, hop 441)
    audio = torch.randn(2 * B, (FRAMES - 1) * 441, device="cuda", generator=gen)
    win = msst.hann_window(2048)
    out = {}
    f_split = 2.0 * rows * ftot * DIM
    f_mask = 2.0 * rows * nb * DIM * hid + 2.0 * rows * hid * 2 * ftot
    for name, fn, flops, nbytes in (
            ("band_split", lambda: plan.band_split(x, out=feats), f_split,
             4 * rows * ftot + 4 * rows * nb * DIM + 2 * DIM * ftot),
            ("mask_estimator", lambda: plan.mask_estimator(feats, out=m), f_mask,
             4 * rows * nb * DIM + 4 * rows * ftot + 2 * nb * hid * (DIM + 2 * 2 * ftot // nb)),
            ("band_gather", lambda: plan.band_gather(stft, B), 0, 8 * rows * ftot),
            ("mask_merge", lambda: plan.mask_merge(masks, stft, B), 0, 12 * rows * ftot),
            ("stft", lambda: msst.stft(audio, 2048, 441, win), 0,
             4 * audio.numel() + 8 * 2 * B * 1025 * FRAMES),
            ("istft", lambda: msst.istft(stft, 2048, 441, win, length=audio.shape[1]), 0,
             8 * 2 * B * 1025 * FRAMES + 4 * audio.numel())):
        fn()
        us = time_events(torch, fn, 50) / 50 * 1e3
        e = {"us": round(us, 2), "gbs": round(nbytes / (us * 1e-6) / 1e9, 1)}
        if flops:
            tf = flops / (us * 1e-6) / 1e12
            e.update({"tflops": round(tf, 1), "frac_mfma": round(tf / PEAK_F16_TFLOPS, 4)})
        out[name] = e
    out["config"] = f"BSRoformer bands: 62 bands, features {ftot}, rows {rows}, dim {DIM}, " \
                    f"MLP {DIM}->{hid}->2*band, fp16 weights, fp32 input; STFT side: " \
                    f"stereo, 1025 bins, {FRAMES} frames, one stem; STFT / iSTFT of 8 s " \
                    f"stereo at 44.1 kHz, n_fft 2048, hop 441, fp32"
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=1, help="chunks per step (the batch-of-4 report uses 4)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the other configurations' sections (batch of 4 chunks, fp32 "
                         "layer, GEMM sweep)")
    ap.add_argument("--pmc-sample", nargs="?", const="ff1", choices=("ff1", "kernels"),
                    help="run only the copy-kernel calibration and then the FF1 GEMM (ff1) or "
                         "every kernel of one transformer (kernels), 3 launches each, for "
                         "rocprofv3 --pmc passes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(chunks are independent: several GPUs would each run their own chunks).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    msst = load_msst()
    msst.lib()
    torch.manual_seed(0)
    B = args.batch
    if args.pmc_sample:
        pmc_sample(msst, torch, B, args.pmc_sample)
        return
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

    # Host-buffer rate: pinned host chunk -> device, stack, device -> host.
    xh = torch.empty(B, FRAMES, BANDS, DIM, pin_memory=True)
    xh.copy_(x.cpu())

    def pcie_step():
        x.copy_(xh, non_blocking=True)
        st(x)
        xh.copy_(x, non_blocking=True)
    pcie_step()
    pcie_ms = time_events(torch, pcie_step, 5) / 5 / B

    # GEMM replay: the stack's GEMM launches alone.
    run = gemm_replay(msst, torch, layers, B)
    run()
    reps = max(2, min(5, args.steps))
    gemm_ms = time_events(torch, run, reps) / reps
    M = B * FRAMES * BANDS
    gemm_flops = gemm_flops_per_token_layer() * M * 2 * DEPTH
    gemm_tflops = gemm_flops / (gemm_ms * 1e-3) / 1e12

    # Dominant kernel: FF1 GEMM (bias + GELU, fp16 out).
    xn, hid, w1, b1 = ff1_inputs(torch, layers, M)
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
        "pcie_inclusive_ms_per_chunk": round(pcie_ms, 3),
        "gemm_ms_per_chunk": round(gemm_ms / B, 3),
        "gemm_tflops": round(gemm_tflops, 1),
        "gemm_frac_of_peak": round(gemm_tflops / PEAK_F16_TFLOPS, 4),
        "stack_tflops": round((gemm_flops + attn_flops_chunk(B)) / (ms_per_step * 1e-3) / 1e12, 1),
        "roofline": {
            "kernel": f"gemm_pp_kernel<32,3,plain,GELU,half> FF1 M={M} "
                      "K=512 N=2048 bias+GELU fp16 out",
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
    out["kernels"] = kernel_table(msst, torch, layers, B)
    # Either side of the stack (not part of the timed step): band split and
    # one stem's mask estimator on the same chunk.
    out["bands"] = band_table(msst, torch, B)
    out["mbr_stack"] = mbr_stack_time(msst, torch, max(2, min(10, args.steps)))
    if not args.no_configs:
        out["config5_batch4"] = batch4_stack(msst, torch, layers, final_gamma,
                                             max(2, min(5, args.steps)))
        out["config1_fp32_layer"] = fp32_mbr_time_layer(msst, torch)
        out["config2_gemm_sweep"] = gemm_sweep(msst, torch)
    if not args.no_cpu:
        cpu, parity = cpu_baseline_and_parity(msst, torch, args)
        out["cpu_baseline"] = cpu
        out["parity"] = parity
    print(json.dumps(out))


if __name__ == "__main__":
    main()
