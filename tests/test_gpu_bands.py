"""Band split and mask estimator (grouped over bands) against the CPU oracle.

The oracle runs the reference's per-band loop (model_bs_roformer.cu:337-414)
in fp32 on the fp16-rounded weights; the HIP path rounds the normalised
bands and the hidden activations to fp16 (the reference's ops::linear casts
its input to fp16), so the tolerance is the fp16 one, normwise per band.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from conftest import TOL_F16, rel_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

# BSRoformer's 62 bands (1025 STFT bins), stereo: 2 * freqs * 2 features.
BSR_FREQS = [2] * 24 + [4] * 12 + [12] * 8 + [24] * 8 + [48] * 8 + [128, 129]
BSR_DIMS = [4 * f for f in BSR_FREQS]


def dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    return t if dtype is None else t.to(dtype)


def host(t):
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def r16(a):
    return a.astype(np.float16).astype(np.float32)


def split_weights(dims, dim, seed):
    rng = np.random.default_rng(seed)
    g = [(1.0 + 0.02 * rng.standard_normal(d)).astype(np.float32) for d in dims]
    w = [r16((rng.standard_normal((dim, d)) / math.sqrt(d)).astype(np.float32)) for d in dims]
    b = [(0.02 * rng.standard_normal(dim)).astype(np.float32) for d in dims]
    return g, w, b


def mask_weights(dims, dim, hid, L, seed):
    rng = np.random.default_rng(seed)
    ws, bs = [], []
    for d in dims:
        wl, bl, K = [], [], dim
        for l in range(L):
            N = 2 * d if l == L - 1 else hid
            wl.append(r16((rng.standard_normal((N, K)) / math.sqrt(K)).astype(np.float32)))
            bl.append((0.02 * rng.standard_normal(N)).astype(np.float32))
            K = N
        ws.append(wl)
        bs.append(bl)
    return ws, bs


def per_band_err(y, r, dims):
    off = np.concatenate([[0], np.cumsum(dims)])
    return max(rel_err(y[:, off[i]:off[i + 1]], r[:, off[i]:off[i + 1]]) for i in range(len(dims)))


CASES = [
    ("bsr", 801, BSR_DIMS, 512, 2048, 2),
    ("small-L1", 37, [4, 8, 36, 130, 2], 64, 0, 1),
    ("small-L2", 130, [6, 64, 66, 128, 200, 1024], 128, 192, 2),
    ("small-L3", 257, [8, 16, 48], 64, 128, 3),
]


@pytest.mark.parametrize("name,rows,dims,dim,hid,L", CASES, ids=[c[0] for c in CASES])
def test_band_split(msst, oracle, cuda, name, rows, dims, dim, hid, L):
    rng = np.random.default_rng(rows + dim)
    x = rng.standard_normal((rows, sum(dims))).astype(np.float32)
    g, w, b = split_weights(dims, dim, 7)
    plan = msst.BandPlan(dims, dim, split=([dev(a) for a in g], [dev(a, torch.float16) for a in w],
                                           [dev(a) for a in b]))
    y = host(plan.band_split(dev(x)))
    r = oracle.band_split(x, dims, g, w, b)
    assert y.shape == (rows, len(dims), dim)
    errs = [rel_err(y[:, i], r[:, i]) for i in range(len(dims))]
    assert max(errs) < TOL_F16, (int(np.argmax(errs)), max(errs))


@pytest.mark.parametrize("name,rows,dims,dim,hid,L", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("xdt", ["f32", "f16"])
def test_mask_estimator(msst, oracle, cuda, name, rows, dims, dim, hid, L, xdt):
    rng = np.random.default_rng(rows + 3 * dim)
    x = rng.standard_normal((rows, len(dims), dim)).astype(np.float32)
    if xdt == "f16":
        x = r16(x)
    ws, bs = mask_weights(dims, dim, hid, L, 11)
    plan = msst.BandPlan(dims, dim, mask=([[dev(a, torch.float16) for a in band] for band in ws],
                                          [[dev(a) for a in band] for band in bs]))
    xd = dev(x, torch.float32 if xdt == "f32" else torch.float16)
    y = host(plan.mask_estimator(xd))
    r = oracle.mask_estimator(x, dims, ws, bs)
    assert y.shape == (rows, sum(dims))
    assert per_band_err(y, r, dims) < TOL_F16


def test_band_plan_holds_both_parts_and_is_reusable(msst, oracle, cuda):
    """One plan with the split and the mask estimator, called twice with
    different row counts (the plan carries no per-call state)."""
    dims, dim, hid, L = [4, 8, 12, 24], 64, 128, 2
    g, w, b = split_weights(dims, dim, 1)
    ws, bs = mask_weights(dims, dim, hid, L, 2)
    plan = msst.BandPlan(dims, dim,
                         split=([dev(a) for a in g], [dev(a, torch.float16) for a in w],
                                [dev(a) for a in b]),
                         mask=([[dev(a, torch.float16) for a in band] for band in ws],
                               [[dev(a) for a in band] for band in bs]))
    for rows in (300, 17):
        x = np.random.default_rng(rows).standard_normal((rows, sum(dims))).astype(np.float32)
        feats = plan.band_split(dev(x))
        m = host(plan.mask_estimator(feats))
        rf = oracle.band_split(x, dims, g, w, b)
        rm = oracle.mask_estimator(rf, dims, ws, bs)
        assert per_band_err(m, rm, dims) < TOL_F16


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_tanh_and_glu(msst, oracle, cuda, dt):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((333, 2 * 129)) * 3).astype(np.float32)
    tdt = torch.float32 if dt == "f32" else torch.float16
    if dt == "f16":
        x = r16(x)
    tol = 1e-6 if dt == "f32" else 1e-3
    t = host(msst.tanh(dev(x, tdt)))
    assert rel_err(t, oracle.activation(x, "tanh")) < tol
    g = host(msst.glu(dev(x, tdt)))
    assert g.shape == (333, 129)
    assert rel_err(g, oracle.glu(x)) < tol


def _mel_like(F, ch, nb, seed):
    """Overlapping contiguous bin ranges (as mel filters > 0 give), stereo
    doubled (model_mel_band_roformer.cu:238-268)."""
    rng = np.random.default_rng(seed)
    edges = np.sort(rng.choice(np.arange(1, F - 1), nb - 1, replace=False))
    lo = np.concatenate([[0], edges - 2])
    hi = np.concatenate([edges + 2, [F - 1]])
    fidx, dims = [], []
    for a, b in zip(lo, hi):
        bins = np.arange(max(a, 0), min(b, F - 1) + 1)
        fidx.extend([int(f) * ch + s for f in bins for s in range(ch)])
        dims.append(2 * len(bins) * ch)
    return fidx, dims


STFT_CASES = [("bsr", 1, 2, 1025, 801, 1, None), ("bsr-2stem", 2, 2, 1025, 130, 2, None),
              ("mbr", 1, 2, 1025, 801, 1, 60), ("mbr-mono-3stem", 2, 1, 257, 70, 3, 20)]


@pytest.mark.parametrize("name,B,ch,F,T,stems,mel", STFT_CASES, ids=[c[0] for c in STFT_CASES])
def test_band_gather_and_mask_merge(msst, oracle, cuda, name, B, ch, F, T, stems, mel):
    rng = np.random.default_rng(F + T)
    if mel:
        fidx, dims = _mel_like(F, ch, mel, 3)
    else:
        fidx, dims = None, [4 * f for f in BSR_FREQS] if (ch == 2 and F == 1025) else [2 * ch] * F
    plan = msst.BandPlan(dims, 64, channels=ch, stft_bins=F, freq_indices=fidx)
    stft = rng.standard_normal((B * ch, F, T, 2)).astype(np.float32)
    feats = host(plan.band_gather(dev(stft), B))
    np.testing.assert_array_equal(feats, oracle.band_gather(stft, B, fidx))
    masks = rng.standard_normal((stems, B, T, sum(dims))).astype(np.float32)
    for zero_dc in (True, False):
        y = host(plan.mask_merge(dev(masks), dev(stft), B, zero_dc))
        r = oracle.mask_merge(masks, stft, B, fidx, zero_dc)
        assert y.shape == r.shape
        assert rel_err(y, r) < 1e-6
