"""Layer- and stack-level parity of the HIP Roformer path against the CPU
oracle, on the workloads the benchmark reports:

  MelBandRoformer time layer, fp32, x [60, 801, 384]      (full size)
  MelBandRoformer stack, fp16, dim 384, [60 bands, 801]   (depth 1 and the full
                                                          depth 6 at full size vs
                                                          the oracle; properties)
  BSRoformer stack, fp16, dim 512, [62 bands, 801]        (depth 1 and the full
                                                          depth 12 at full size vs
                                                          the oracle; properties)
  BSRoformer, batch of 4 chunks                           (batch consistency:
                                                          bit-identical to 4
                                                          single-chunk runs)
Weights: matrices and biases ~ N(0, 0.02), gammas 1 + N(0, 0.02), x ~ N(0,1).
"""
from __future__ import annotations

import numpy as np
import pytest

import torch_ref as R
from conftest import TOL_F16, TOL_F32, rel_err

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

MATS = ("w_qkv", "w_gate", "w_out", "w_ff1", "w_ff2")


def make_layers(seed, n, dim, heads, ff, fp16, final_norm):
    rng = np.random.default_rng(seed)
    layers = [R.random_layer(rng, dim, heads, 64, ff, final_norm=final_norm) for _ in range(n)]
    if fp16:
        for w in layers:
            for m in MATS:
                w[m] = w[m].astype(np.float16).astype(np.float32)
    return layers


def upload(layers, fp16):
    out = []
    for w in layers:
        d = {}
        for k, v in w.items():
            if v is None:
                continue
            t = torch.from_numpy(np.ascontiguousarray(v)).cuda()
            if fp16 and k in MATS:
                t = t.half()
            d[k] = t
        out.append(d)
    return out


def build_stack(msst, layers, fp16, B, T, F, dim, heads, ff, final_gamma=None):
    dl = upload(layers, fp16)
    fg = None if final_gamma is None else torch.from_numpy(final_gamma).cuda()
    st = msst.RoformerStack(dl, fg, B, T, F, dim, heads, 64, ff, msst.F16 if fp16 else msst.F32)
    st._keep = dl
    return st


def run_stack(msst, oracle, B, T, F, dim, heads, ff, depth, fp16, mbr, seed=0):
    layers = make_layers(seed, 2 * depth, dim, heads, ff, fp16, final_norm=mbr)
    rng = np.random.default_rng(seed + 99)
    fg = None if mbr else (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    x = rng.standard_normal((B, T, F, dim)).astype(np.float32)
    st = build_stack(msst, layers, fp16, B, T, F, dim, heads, ff, fg)
    xd = torch.from_numpy(x).cuda()
    st(xd)
    torch.cuda.synchronize()
    y = xd.cpu().numpy()
    r = oracle.roformer_stack(x, [oracle.LayerWeights(**w) for w in layers], heads, 64, fg)
    return rel_err(y, r)


@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("mbr", [False, True])
@pytest.mark.parametrize("B,T,F,dim,heads,ff,depth", [(1, 70, 5, 128, 2, 512, 2),
                                                      (2, 33, 7, 192, 3, 256, 1),
                                                      (1, 130, 62, 128, 2, 256, 1)])
def test_stack_small(msst, oracle, cuda, B, T, F, dim, heads, ff, depth, fp16, mbr):
    e = run_stack(msst, oracle, B, T, F, dim, heads, ff, depth, fp16, mbr)
    assert e < (TOL_F16 if fp16 else TOL_F32), e


def test_mbr_time_layer_fp32_full_size(msst, oracle, cuda):
    """Single MelBandRoformer time layer, fp32, x [60, 801, 384], N(0,1)."""
    F, T, dim, heads, ff = 60, 801, 384, 8, 1536
    layers = make_layers(0, 2, dim, heads, ff, False, final_norm=False)
    x = np.random.default_rng(0).standard_normal((F, T, dim)).astype(np.float32)
    st = build_stack(msst, layers, False, 1, T, F, dim, heads, ff)
    xd = torch.from_numpy(x).cuda()
    st.transformer(xd, 0, 0)
    torch.cuda.synchronize()
    c, s = oracle.rope_table(T, 64)
    r = oracle.transformer(x, oracle.LayerWeights(**layers[0]), c, s, heads, 64)
    e = rel_err(xd.cpu().numpy(), r)
    assert e < TOL_F32, e


@pytest.mark.parametrize("name,F,dim,ff,mbr", [("bsr", 62, 512, 2048, False),
                                               ("mbr", 60, 384, 1536, True)])
def test_full_size_depth1_fp16(msst, oracle, cuda, name, F, dim, ff, mbr):
    """Both stacks at full spatial size, one depth (time + freq layer)."""
    e = run_stack(msst, oracle, 1, 801, F, dim, 8, ff, 1, True, mbr, seed=4)
    assert e < TOL_F16, e


@pytest.mark.parametrize("name,F,dim,ff,depth,mbr", [("bsr", 62, 512, 2048, 12, False),
                                                     ("mbr", 60, 384, 1536, 6, True)])
def test_full_depth_against_oracle(msst, oracle, cuda, name, F, dim, ff, depth, mbr):
    """Configs 4 and 3 at full size and full depth against the oracle: the
    12-depth BSRoformer stack with its final norm on [1, 801, 62, 512], the
    6-depth MelBandRoformer stack with a norm closing every transformer on
    [1, 801, 60, 384]; fp16 weights, fp32 residual."""
    print(f"full-depth {name}: depth {depth}, [1, 801, {F}, {dim}]", flush=True)
    e = run_stack(msst, oracle, 1, 801, F, dim, 8, ff, depth, True, mbr, seed=7)
    print(f"full-depth {name}: max rel err {e:.3e}", flush=True)
    assert e < TOL_F16, e


@pytest.mark.parametrize("fp16", [False, True])
@pytest.mark.parametrize("mbr", [False, True])
def test_stack_layer_schedule_against_oracle(msst, oracle, cuda, fp16, mbr):
    """msst_roformer_stack_layer driven through the depth loop's switches:
    time/freq_transformer_depth 2 and skip_connection (the skip sums as
    torch adds between calls), against the oracle's restatement of
    model_bs_roformer.cu:477-539."""
    B, T, F, dim, heads, ff, depth, td, fd = 1, 40, 9, 128, 2, 256, 3, 2, 2
    per = td + fd
    rng = np.random.default_rng(31)
    layers = [R.random_layer(rng, dim, heads, 64, ff, final_norm=mbr and (i % per in (td - 1, per - 1)))
              for i in range(depth * per)]
    if fp16:
        for w in layers:
            for m in MATS:
                w[m] = w[m].astype(np.float16).astype(np.float32)
    fg = None if mbr else (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    x = rng.standard_normal((B, T, F, dim)).astype(np.float32)
    st = build_stack(msst, layers, fp16, B, T, F, dim, heads, ff)
    xd = torch.from_numpy(x).cuda()
    stored = []
    for d in range(depth):
        for j in range(d):
            xd += stored[j]
        for i in range(per):
            st.layer(xd, d * per + i, 0 if i < td else 1)
        stored.append(xd.clone())
    if fg is not None:
        xd = msst.rms_norm(xd, torch.from_numpy(fg).cuda(), float(np.sqrt(dim)))
    torch.cuda.synchronize()
    r = oracle.roformer_stack_schedule(x, [oracle.LayerWeights(**w) for w in layers], heads, 64,
                                       fg, td, fd, True)
    e = rel_err(xd.cpu().numpy(), r)
    assert e < (TOL_F16 if fp16 else TOL_F32), e


@pytest.mark.parametrize("name,F,dim,ff,depth,mbr", [("bsr", 62, 512, 2048, 12, False),
                                                     ("mbr", 60, 384, 1536, 6, True)])
def test_full_depth_properties(msst, cuda, name, F, dim, ff, depth, mbr):
    """Both stacks at full depth: finite, deterministic, and the batch-of-4
    run equals four single-chunk runs bit for bit — every
    kernel's per-row / per-sequence arithmetic is independent of the batch."""
    T, heads = 801, 8
    layers = make_layers(5, 2 * depth, dim, heads, ff, True, final_norm=mbr)
    rng = np.random.default_rng(6)
    fg = None if mbr else (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    x = torch.from_numpy(rng.standard_normal((4, T, F, dim)).astype(np.float32)).cuda()
    st4 = build_stack(msst, layers, True, 4, T, F, dim, heads, ff, fg)
    st1 = build_stack(msst, layers, True, 1, T, F, dim, heads, ff, fg)
    y4 = st4(x.clone())
    singles = [st1(x[i:i + 1].clone()) for i in range(4)]
    again = st1(x[0:1].clone())
    torch.cuda.synchronize()
    assert torch.isfinite(y4).all()
    for i in range(4):
        assert torch.equal(y4[i:i + 1], singles[i]), i
    assert torch.equal(again, singles[0])
    # the stack changed the input substantially (it is not an identity)
    assert (y4 - x).abs().max().item() > 0.1


@pytest.mark.parametrize("fp16", [True, False])
def test_stack_graph_capture_replays(msst, cuda, fp16):
    """The stack launches kernels only (no allocation, memset or host
    synchronisation), so a caller can capture it in a HIP graph.  Every replay,
    with eager stack work and synchronisations between them, must equal the
    eager result bit for bit (full-size BSRoformer chunk, depth 2)."""
    T, F, dim, heads, ff, depth = 801, 62, 512, 8, 2048, 2
    layers = make_layers(11, 2 * depth, dim, heads, ff, fp16, final_norm=False)
    rng = np.random.default_rng(12)
    fg = (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    x0 = torch.from_numpy(rng.standard_normal((1, T, F, dim)).astype(np.float32)).cuda()
    st = build_stack(msst, layers, fp16, 1, T, F, dim, heads, ff, fg)
    ref = st(x0.clone())
    torch.cuda.synchronize()
    xg = x0.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        st(xg)  # first launch of every kernel outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st(xg)
    torch.cuda.synchronize()
    other = x0.clone()
    for _ in range(3):
        xg.copy_(x0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(xg, ref)
        st(other)  # eager work between replays
        torch.cuda.synchronize()
