"""msst_roformer_stack_noalloc (the library's static device scratch, no
allocation) against msst_roformer_stack (caller workspace) through the C ABI:
two calls in a row, the second with a smaller stack, bit-identical to the
workspace entry point on the same weights and input."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _stack(msst, seed, B, T, F, dim, depth, ff, per_layer_norm):
    g = torch.Generator(device="cuda").manual_seed(seed)
    H, Dh = 8, 64
    hd = H * Dh

    def n(*s, dt=torch.float16):
        return (torch.randn(*s, device="cuda", generator=g) * 0.02).to(dt)

    def gm():
        return 1.0 + torch.randn(dim, device="cuda", generator=g) * 0.02

    layers = []
    for _ in range(2 * depth):
        lw = dict(attn_gamma=gm(), w_qkv=n(3 * hd, dim), w_gate=n(H, dim),
                  b_gate=n(H, dt=torch.float32), w_out=n(dim, hd), ff_gamma=gm(),
                  w_ff1=n(ff, dim), b_ff1=n(ff, dt=torch.float32), w_ff2=n(dim, ff),
                  b_ff2=n(dim, dt=torch.float32))
        if per_layer_norm:
            lw["final_gamma"] = gm()
        layers.append(lw)
    fg = None if per_layer_norm else gm()
    st = msst.RoformerStack(layers, fg, B, T, F, dim, H, Dh, ff, msst.F16)
    x = torch.randn(B, T, F, dim, device="cuda", generator=g)
    return st, x


@pytest.mark.parametrize("order", ["large_then_small"])
def test_stack_noalloc_matches_workspace_entry(msst, order):
    cases = [  # (seed, B, T, F, dim, depth, ff, MelBandRoformer-style norms)
        (11, 1, 161, 62, 512, 2, 2048, False),   # 9982 tokens: ~61.7 MB of scratch
        (12, 1, 96, 12, 384, 1, 1536, True),     # smaller, second call
    ]
    for seed, B, T, F, dim, depth, ff, pln in cases:
        st, x = _stack(msst, seed, B, T, F, dim, depth, ff, pln)
        need = msst.lib().msst_roformer_stack_workspace(st.desc)
        assert 0 < need <= msst.STACK_SCRATCH_BYTES, need
        print(f"noalloc case B={B} T={T} F={F} dim={dim} depth={depth}: "
              f"scratch {need} bytes", flush=True)
        ref = x.clone()
        st(ref)
        got = x.clone()
        st.call_noalloc(got)
        torch.cuda.synchronize()
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref), float((got - ref).abs().max())


def test_stack_noalloc_graph_capture(msst):
    """The callers this entry point is for include code under HIP graph
    capture: a captured call replays three times, with eager calls of both
    entry points between the replays, each bit-identical to the workspace
    entry point."""
    st, x = _stack(msst, 14, 1, 161, 62, 512, 2, 2048, False)
    ref = x.clone()
    st(ref)
    xg = x.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        st.call_noalloc(xg)  # first launches outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st.call_noalloc(xg)
    torch.cuda.synchronize()
    for _ in range(3):
        xg.copy_(x)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(xg, ref), float((xg - ref).abs().max())
        st(x.clone())
        st.call_noalloc(x.clone())
        torch.cuda.synchronize()


def test_stack_noalloc_rejects_oversized_stack(msst):
    st, x = _stack(msst, 13, 1, 801, 62, 512, 1, 2048, False)  # ~307 MB of workspace
    assert msst.lib().msst_roformer_stack_workspace(st.desc) > msst.STACK_SCRATCH_BYTES
    before = x.clone()
    with pytest.raises(msst.MsstError, match="scratch"):
        st.call_noalloc(x)
    torch.cuda.synchronize()
    assert torch.equal(x, before)
