"""Pins the C oracle (oracle/msst_oracle.c) before it is trusted as the
parity checker of the HIP path.

Each oracle function is checked against something it does not share code
with: numpy/torch library routines in float64, closed forms, invariants of
the mathematics and brute force on tiny inputs — chosen so a dropped term,
a wrong sign or index, or a transposed operand fails at least one check.
The reference itself (CUDA + cuBLAS) cannot be built or run here and holds
no golden vectors, so these are the pins.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import torch_ref as R
from conftest import rel_err

RNG = np.random.default_rng(1234)


def rnd(*shape, s=1.0):
    return (RNG.standard_normal(shape) * s).astype(np.float32)


# --------------------------------------------------------------------- linear
@pytest.mark.parametrize("M,K,N", [(1, 1, 1), (7, 5, 3), (13, 96, 50), (37, 130, 17),
                                   (64, 384, 96)])
@pytest.mark.parametrize("act", ["none", "gelu", "sigmoid", "silu"])
def test_linear_matches_float64_library(oracle, M, K, N, act):
    x, w, b = rnd(M, K), rnd(N, K, s=0.02), rnd(N, s=0.02)
    y = oracle.linear(x, w, b, act)
    r = R.linear(x, w, b, act).numpy()
    assert rel_err(y, r) < 1e-6


def test_linear_residual_and_no_bias(oracle):
    x, w, res = rnd(9, 40), rnd(11, 40), rnd(9, 11)
    y = oracle.linear(x, w, None, "none", residual=res)
    r = x.astype(np.float64) @ w.T.astype(np.float64) + res
    assert rel_err(y, r) < 1e-6


def test_linear_identity_and_selection(oracle):
    x = rnd(10, 16)
    np.testing.assert_array_equal(oracle.linear(x, np.eye(16, dtype=np.float32)), x)
    perm = RNG.permutation(16)[:5]
    sel = np.eye(16, dtype=np.float32)[perm]          # W rows are one-hot
    np.testing.assert_array_equal(oracle.linear(x, sel), x[:, perm])
    b = rnd(5)
    y = oracle.linear(np.zeros((3, 16), np.float32), sel, b)
    np.testing.assert_array_equal(y, np.broadcast_to(b, (3, 5)))


# ---------------------------------------------------------------- activations
def test_activation_closed_forms(oracle):
    z = np.zeros(4, np.float32)
    assert np.all(oracle.activation(z, "gelu") == 0.0)
    assert np.all(oracle.activation(z, "sigmoid") == 0.5)
    x = np.linspace(-8, 8, 101).astype(np.float32)
    s = oracle.activation(x, "sigmoid")
    np.testing.assert_allclose(s + oracle.activation(-x, "sigmoid"), 1.0, atol=1e-6)
    big = np.array([10.0, 20.0], np.float32)
    np.testing.assert_allclose(oracle.activation(big, "gelu"), big, rtol=1e-6)
    np.testing.assert_allclose(oracle.activation(-big, "gelu"), 0.0, atol=1e-6)
    np.testing.assert_allclose(oracle.activation(x, "silu"), x * s, rtol=2e-6, atol=1e-7)


# ------------------------------------------------------------------- rms_norm
@pytest.mark.parametrize("rows,D", [(1, 1), (5, 7), (33, 384), (8, 512), (3, 1100)])
def test_rms_norm_matches_normalize(oracle, rows, D):
    x, g = rnd(rows, D), (1 + rnd(D, s=0.02))
    y = oracle.rms_norm(x, g, math.sqrt(D))
    r = R.rms_norm(x, g, math.sqrt(D)).numpy()
    assert rel_err(y, r) < 1e-6


def test_rms_norm_closed_forms(oracle):
    D = 64
    g = np.ones(D, np.float32)
    for c in (0.5, -3.0, 100.0):
        y = oracle.rms_norm(np.full((1, D), c, np.float32), g, math.sqrt(D))
        np.testing.assert_allclose(y, np.sign(c), rtol=1e-6)
    x = rnd(4, D)
    np.testing.assert_allclose(oracle.rms_norm(7.5 * x, g, 2.0), oracle.rms_norm(x, g, 2.0),
                               rtol=2e-6, atol=1e-7)
    y = oracle.rms_norm(x, g, math.sqrt(D))
    np.testing.assert_allclose(np.sum(y.astype(np.float64) ** 2, -1), D, rtol=1e-5)
    # epsilon lives inside the sqrt: a zero row stays finite and zero
    assert np.all(oracle.rms_norm(np.zeros((1, D), np.float32), g, 1.0) == 0.0)


# ----------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("n,dh", [(1, 64), (62, 64), (801, 64), (9, 16)])
def test_rope_table_geometry(oracle, n, dh):
    c, s = oracle.rope_table(n, dh)
    assert c.shape == (n, dh // 2)
    np.testing.assert_allclose(c.astype(np.float64) ** 2 + s.astype(np.float64) ** 2, 1.0,
                               atol=1e-6)
    np.testing.assert_array_equal(c[0], 1.0)
    np.testing.assert_array_equal(s[0], 0.0)
    ang = R.rope_angles(n, dh).numpy()
    # float32 angle n*freq carries ~n*ulp error; compare on the circle
    err = np.abs(np.angle(np.exp(1j * ang) * (c - 1j * s)))
    assert err.max() < 1e-6 * max(n, 1) + 1e-6
    # i = 0 rotates by exactly one radian per position
    np.testing.assert_allclose(c[:, 0], np.cos(np.arange(n, dtype=np.float32)), atol=1e-6)


def test_rope_apply_matches_complex_rotation(oracle):
    B, H, N, D = 2, 3, 11, 16
    q, k = rnd(B, H, N, D), rnd(B, H, N, D)
    c, s = oracle.rope_table(N, D)
    qr, kr = oracle.rope_apply(q, k, c, s)
    ang = torch.as_tensor(np.arctan2(s, c), dtype=torch.float64)
    assert rel_err(qr, R.rope(q, ang).numpy()) < 1e-6
    assert rel_err(kr, R.rope(k, ang).numpy()) < 1e-6
    np.testing.assert_array_equal(qr[:, :, 0], q[:, :, 0])  # position 0 is identity
    pair = lambda a: np.sqrt(a[..., 0::2] ** 2 + a[..., 1::2] ** 2)
    np.testing.assert_allclose(pair(qr), pair(q), rtol=1e-5)


def test_rope_relative_position(oracle):
    """<R_m q, R_n k> depends only on m - n."""
    D, N = 16, 20
    base_q, base_k = rnd(D), rnd(D)
    q = np.broadcast_to(base_q, (1, 1, N, D)).copy()
    k = np.broadcast_to(base_k, (1, 1, N, D)).copy()
    c, s = oracle.rope_table(N, D)
    qr, kr = oracle.rope_apply(q, k, c, s)
    dots = qr[0, 0] @ kr[0, 0].T
    for off in (-3, 0, 5):
        diag = np.diagonal(dots, offset=off)
        np.testing.assert_allclose(diag, diag[0], rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------ attention
@pytest.mark.parametrize("B,H,N,Nk,D", [(1, 1, 1, 1, 8), (2, 3, 17, 19, 32), (1, 2, 62, 62, 64),
                                        (1, 1, 129, 70, 64)])
def test_attention_matches_sdpa(oracle, B, H, N, Nk, D):
    q, k, v = rnd(B, H, N, D), rnd(B, H, Nk, D), rnd(B, H, Nk, D)
    y = oracle.attention(q, k, v)
    assert rel_err(y, R.attention(q, k, v).numpy()) < 1e-6


def test_attention_closed_forms(oracle):
    B, H, N, D = 1, 2, 9, 16
    v = rnd(B, H, N, D)
    q0 = np.zeros((B, H, N, D), np.float32)
    y = oracle.attention(q0, rnd(B, H, N, D), v)
    np.testing.assert_allclose(y, np.broadcast_to(v.mean(2, keepdims=True), y.shape), rtol=1e-5,
                               atol=1e-6)
    # one very peaked key per query selects that key's value row
    k = np.eye(N, D, dtype=np.float32)[None, None].repeat(H, 1) * 50.0
    qs = k.copy()
    y = oracle.attention(qs, k, v, scale=1.0)
    np.testing.assert_allclose(y, v, rtol=1e-5, atol=1e-5)


# -------------------------------------------------------- head split / merge
def test_split_and_merge_index_identities(oracle):
    B, N, H, D = 2, 5, 3, 4
    qkv = np.arange(B * N * 3 * H * D, dtype=np.float32).reshape(B, N, 3 * H * D)
    q, k, v = oracle.split_qkv(qkv, H, D)
    r = qkv.reshape(B, N, 3, H, D).transpose(2, 0, 3, 1, 4)
    np.testing.assert_array_equal(q, r[0])
    np.testing.assert_array_equal(k, r[1])
    np.testing.assert_array_equal(v, r[2])
    gates = (np.arange(B * N * H, dtype=np.float32).reshape(B, N, H) + 1) / 7
    m = oracle.gate_merge(q, gates)
    exp = (q * gates.transpose(0, 2, 1)[..., None]).transpose(0, 2, 1, 3).reshape(B, N, H * D)
    np.testing.assert_array_equal(m, exp)


# ---------------------------------------------------------- layer and stack
@pytest.mark.parametrize("final", [False, True])
def test_transformer_matches_torch_composition(oracle, final):
    rng = np.random.default_rng(7)
    B, N, dim, H, Dh, ff = 3, 13, 32, 2, 16, 64
    w = R.random_layer(rng, dim, H, Dh, ff, final_norm=final)
    x = rng.standard_normal((B, N, dim)).astype(np.float32)
    c, s = oracle.rope_table(N, Dh)
    y = oracle.transformer(x, oracle.LayerWeights(**w), c, s, H, Dh)
    ang = torch.as_tensor(np.arctan2(s, c), dtype=torch.float64)
    r = R.transformer(x, w, H, Dh, ang).numpy()
    assert rel_err(y, r) < 2e-6


def test_stack_matches_torch_composition(oracle):
    rng = np.random.default_rng(11)
    B, T, Fb, dim, H, Dh, ff, depth = 2, 9, 5, 32, 2, 16, 64, 2
    layers = [R.random_layer(rng, dim, H, Dh, ff) for _ in range(2 * depth)]
    fg = (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    x = rng.standard_normal((B, T, Fb, dim)).astype(np.float32)
    y = oracle.roformer_stack(x, [oracle.LayerWeights(**w) for w in layers], H, Dh, fg)
    r = R.stack(x, layers, H, Dh, fg).numpy()
    assert rel_err(y, r) < 5e-6


def test_stack_axis_order_matters(oracle):
    """Swapping the time and frequency transformers changes the result, so
    the axis-order pin above is not vacuous."""
    rng = np.random.default_rng(3)
    B, T, Fb, dim, H, Dh, ff = 1, 6, 4, 32, 2, 16, 64
    layers = [R.random_layer(rng, dim, H, Dh, ff) for _ in range(2)]
    x = rng.standard_normal((B, T, Fb, dim)).astype(np.float32)
    a = oracle.roformer_stack(x, [oracle.LayerWeights(**w) for w in layers], H, Dh)
    b = oracle.roformer_stack(x, [oracle.LayerWeights(**w) for w in layers[::-1]], H, Dh)
    assert rel_err(a, b) > 1e-3


# ------------------------------------------------ band split / mask estimator
BSR_FREQS = [2] * 24 + [4] * 12 + [12] * 8 + [24] * 8 + [48] * 8 + [128, 129]


def test_tanh_and_glu_closed_forms(oracle):
    x = np.linspace(-20, 20, 4001, dtype=np.float32)
    t = oracle.activation(x, "tanh")
    np.testing.assert_allclose(t, np.tanh(x.astype(np.float64)), rtol=2e-7, atol=1e-7)
    assert t[2000] == 0.0 and np.all(t[:-1] <= t[1:]) and np.array_equal(t, -t[::-1])
    a = rnd(9, 5)
    # zero gate -> half of the value; large gate -> the value; order of halves
    np.testing.assert_array_equal(oracle.glu(np.concatenate([a, np.zeros_like(a)], 1)), a * 0.5)
    np.testing.assert_allclose(oracle.glu(np.concatenate([a, np.full_like(a, 40.0)], 1)), a,
                               rtol=1e-7)
    g = rnd(9, 5)
    r = a.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    assert rel_err(oracle.glu(np.concatenate([a, g], 1)), r) < 1e-6


def _split_weights(dims, dim, seed=3):
    rng = np.random.default_rng(seed)
    gam = [(1.0 + 0.02 * rng.standard_normal(d)).astype(np.float32) for d in dims]
    ws = [(0.02 * rng.standard_normal((dim, d))).astype(np.float32) for d in dims]
    bs = [(0.02 * rng.standard_normal(dim)).astype(np.float32) for d in dims]
    return gam, ws, bs


def test_band_split_single_band_is_norm_then_linear(oracle):
    dims, dim = [24], 16
    x = rnd(11, 24)
    g, w, b = _split_weights(dims, dim)
    y = oracle.band_split(x, dims, g, w, b)
    r = oracle.linear(oracle.rms_norm(x, g[0], math.sqrt(24)), w[0], b[0])
    np.testing.assert_array_equal(y[:, 0, :], r)


def test_band_split_band_independence_and_scale_invariance(oracle):
    dims, dim = [4, 8, 12, 6], 32
    off = np.concatenate([[0], np.cumsum(dims)])
    x = rnd(7, sum(dims))
    g, w, b = _split_weights(dims, dim)
    y = oracle.band_split(x, dims, g, w, b)
    for bi in range(len(dims)):
        x2 = x.copy()
        x2[:, off[bi]:off[bi + 1]] *= 3.5           # rms_norm is scale invariant
        x3 = x.copy()
        x3[:, off[bi]:off[bi + 1]] = rnd(7, dims[bi])  # only band bi changes
        y2 = oracle.band_split(x2, dims, g, w, b)
        y3 = oracle.band_split(x3, dims, g, w, b)
        assert rel_err(y2, y) < 1e-6
        others = [j for j in range(len(dims)) if j != bi]
        np.testing.assert_array_equal(y3[:, others], y[:, others])
        assert not np.allclose(y3[:, bi], y[:, bi])
    # each band equals the single-band split of its own slice
    for bi in range(len(dims)):
        yi = oracle.band_split(x[:, off[bi]:off[bi + 1]], [dims[bi]], [g[bi]], [w[bi]], [b[bi]])
        np.testing.assert_array_equal(yi[:, 0], y[:, bi])


def _mask_weights(dims, dim, hid, L, seed=4):
    rng = np.random.default_rng(seed)
    ws, bs = [], []
    for d in dims:
        wl, bl, K = [], [], dim
        for l in range(L):
            N = 2 * d if l == L - 1 else hid
            wl.append((rng.standard_normal((N, K)) / math.sqrt(K)).astype(np.float32))
            bl.append((0.02 * rng.standard_normal(N)).astype(np.float32))
            K = N
        ws.append(wl)
        bs.append(bl)
    return ws, bs


@pytest.mark.parametrize("L", [1, 2, 3])
def test_mask_estimator_is_per_band_mlp_then_glu(oracle, L):
    dims, dim, hid = [4, 10, 6], 16, 24
    x = rnd(9, len(dims), dim)
    ws, bs = _mask_weights(dims, dim, hid, L)
    y = oracle.mask_estimator(x, dims, ws, bs)
    off = np.concatenate([[0], np.cumsum(dims)])
    for bi, d in enumerate(dims):
        h = x[:, bi]
        for l in range(L):
            h = oracle.linear(h, ws[bi][l], bs[bi][l], "tanh" if l < L - 1 else "none")
        np.testing.assert_array_equal(y[:, off[bi]:off[bi + 1]], oracle.glu(h))
    # float64 restatement of the same network from numpy primitives
    for bi, d in enumerate(dims):
        h = x[:, bi].astype(np.float64)
        for l in range(L):
            h = h @ ws[bi][l].T.astype(np.float64) + bs[bi][l]
            if l < L - 1:
                h = np.tanh(h)
        r = h[:, :d] / (1.0 + np.exp(-h[:, d:]))
        assert rel_err(y[:, off[bi]:off[bi + 1]], r) < 1e-5


def test_mask_estimator_gate_half_selects(oracle):
    """W rows of the gate half set to zero and bias 0 -> sigmoid(0) = 1/2, so
    the mask is half of the value half: a transposed or swapped GLU half fails."""
    dims, dim = [6, 4], 8
    x = rnd(5, 2, dim)
    ws, bs = _mask_weights(dims, dim, 0, 1)
    for bi, d in enumerate(dims):
        ws[bi][0][d:] = 0.0
        bs[bi][0][d:] = 0.0
    y = oracle.mask_estimator(x, dims, ws, bs)
    off = [0, 6, 10]
    for bi, d in enumerate(dims):
        v = oracle.linear(x[:, bi], ws[bi][0][:d], bs[bi][0][:d])
        np.testing.assert_allclose(y[:, off[bi]:off[bi + 1]], 0.5 * v, rtol=1e-6, atol=1e-7)


# ------------------------------------------------------ STFT <-> band features
def _mel_like_fidx(F, ch, nb, seed=0):
    """Overlapping contiguous bin ranges per band (as mel filters > 0 give),
    stereo-doubled the way model_mel_band_roformer.cu:255-268 builds them."""
    rng = np.random.default_rng(seed)
    edges = np.sort(rng.choice(np.arange(1, F - 1), nb - 1, replace=False))
    lo = np.concatenate([[0], edges - 1])
    hi = np.concatenate([edges + 1, [F - 1]])
    fidx, dims = [], []
    for a, b in zip(lo, hi):
        bins = np.arange(max(a, 0), min(b, F - 1) + 1)
        fidx.extend([int(f) * ch + s for f in bins for s in range(ch)])
        dims.append(2 * len(bins) * ch)
    return np.array(fidx, np.int32), dims


@pytest.mark.parametrize("ch", [1, 2])
def test_band_gather_is_stereo_interleave_then_index_select(oracle, ch):
    B, F, T = 2, 9, 5
    stft = rnd(B * ch, F, T, 2)
    # 'b s f t c -> b t (f s) c' with numpy transposes
    ref = stft.reshape(B, ch, F, T, 2).transpose(0, 3, 2, 1, 4).reshape(B, T, F * ch, 2)
    np.testing.assert_array_equal(oracle.band_gather(stft, B), ref.reshape(B, T, -1))
    fidx, _ = _mel_like_fidx(F, ch, 4)
    np.testing.assert_array_equal(oracle.band_gather(stft, B, fidx),
                                  ref[:, :, fidx].reshape(B, T, -1))


@pytest.mark.parametrize("ch", [1, 2])
@pytest.mark.parametrize("zero_dc", [False, True])
def test_mask_merge_matches_scatter_mean_and_complex_product(oracle, ch, zero_dc):
    B, F, T, stems = 2, 11, 6, 2
    fidx, dims = _mel_like_fidx(F, ch, 5, seed=ch)
    n = len(fidx)
    stft = rnd(B * ch, F, T, 2)
    masks = rnd(stems, B, T, 2 * n)
    y = oracle.mask_merge(masks, stft, B, fidx, zero_dc)
    # numpy: complex masks, np.add.at scatter, clamp-divide, complex multiply
    mc = masks[..., 0::2] + 1j * masks[..., 1::2]                   # [stems, B, T, n]
    acc = np.zeros((stems, B, T, F * ch), np.complex128)
    np.add.at(acc, (slice(None), slice(None), slice(None), fidx), mc)
    cnt = np.maximum(np.bincount(fidx, minlength=F * ch).astype(np.float64), 1e-8)
    mean = acc / cnt                                                   # [stems, B, T, g]
    xc = (stft[..., 0] + 1j * stft[..., 1]).reshape(B, ch, F, T)       # [B, s, f, t]
    mg = mean.reshape(stems, B, T, F, ch).transpose(1, 0, 4, 3, 2)     # [B, stems, s, f, t]
    o = xc[:, None] * mg
    if zero_dc:
        o[:, :, :, 0] = 0
    ref = np.stack([o.real, o.imag], -1).reshape(B * stems * ch, F, T, 2)
    assert rel_err(y, ref) < 1e-6


def test_mask_merge_unit_mask_round_trips(oracle):
    """Identity bins (BSRoformer) and a mask of 1 + 0i: the merge returns the
    STFT itself (bin 0 zeroed), so gather and merge invert each other's
    layout changes."""
    B, ch, F, T = 1, 2, 7, 4
    stft = rnd(B * ch, F, T, 2)
    masks = np.zeros((1, B, T, 2 * F * ch), np.float32)
    masks[..., 0::2] = 1.0
    y = oracle.mask_merge(masks, stft, B, None, True)
    ref = stft.copy()
    ref[:, 0] = 0
    np.testing.assert_array_equal(y, ref)
    # the gathered features, conjugated, fed back as the mask: X * conj(X) =
    # |X|^2 on every bin, imaginary part 0
    feats = oracle.band_gather(stft, B)                     # [B, T, 2 * F * ch]
    conj = feats.copy()
    conj[..., 1::2] *= -1.0
    y2 = oracle.mask_merge(conj[None], stft, B, None, False)
    np.testing.assert_allclose(y2[..., 0], (stft ** 2).sum(-1), rtol=1e-6)
    np.testing.assert_allclose(y2[..., 1], 0.0, atol=1e-6)


# ----------------------------------------------------------------- STFT / iSTFT
def _np_stft(x, n_fft, hop, w, center, normalized):
    """torch.stft restated with numpy: reflect pad, frames, window, rfft."""
    if center:
        x = np.pad(x, ((0, 0), (n_fft // 2, n_fft // 2)), mode="reflect")
    T = (x.shape[1] - n_fft) // hop + 1
    idx = np.arange(T)[:, None] * hop + np.arange(n_fft)[None]
    X = np.fft.rfft(x[:, idx].astype(np.float64) * w, axis=-1)        # [B, T, F]
    if normalized:
        X = X / np.sqrt(n_fft)
    return np.stack([X.real, X.imag], -1).transpose(0, 2, 1, 3)      # [B, F, T, 2]


def test_hann_window_is_periodic_hann(oracle):
    for n in (1, 2, 16, 2048):
        ref = np.hanning(n + 1)[:-1] if n > 1 else np.ones(1)
        np.testing.assert_allclose(oracle.hann_window(n), ref, atol=1e-7)


@pytest.mark.parametrize("n_fft,hop,L", [(16, 4, 50), (64, 17, 300), (256, 64, 1000),
                                         (2048, 441, 5000)])
@pytest.mark.parametrize("center", [True, False])
@pytest.mark.parametrize("normalized", [False, True])
def test_stft_matches_numpy_rfft(oracle, n_fft, hop, L, center, normalized):
    x = rnd(2, L)
    w = oracle.hann_window(n_fft)
    y = oracle.stft(x, n_fft, hop, w, center, normalized)
    r = _np_stft(x, n_fft, hop, w.astype(np.float64), center, normalized)
    assert y.shape == r.shape
    assert rel_err(y, r) < 1e-6


def test_stft_closed_forms(oracle):
    """A unit impulse at frame centre with a rectangular window has a flat
    spectrum whose phase turns by -2 pi k n0 / N; a cosine at bin k0 lands
    on bins k0 only (N/2 each side of the real part)."""
    n_fft = 64
    x = np.zeros((1, 200), np.float32)
    x[0, 100] = 1.0
    w = np.ones(n_fft, np.float32)
    y = oracle.stft(x, n_fft, 100, w, center=True)            # frame 1 covers samples 68..131
    n0 = 100 - (100 - n_fft // 2)
    k = np.arange(n_fft // 2 + 1)
    np.testing.assert_allclose(y[0, :, 1, 0], np.cos(-2 * np.pi * k * n0 / n_fft), atol=1e-6)
    np.testing.assert_allclose(y[0, :, 1, 1], np.sin(-2 * np.pi * k * n0 / n_fft), atol=1e-6)
    k0 = 5
    c = np.cos(2 * np.pi * k0 * np.arange(n_fft) / n_fft).astype(np.float32)[None]
    z = oracle.stft(c, n_fft, n_fft, w, center=False)[0, :, 0]
    expect = np.zeros_like(z)
    expect[k0, 0] = n_fft / 2
    np.testing.assert_allclose(z, expect, atol=1e-5)


@pytest.mark.parametrize("n_fft,hop,L", [(64, 16, 400), (256, 100, 3000), (2048, 441, 20000)])
@pytest.mark.parametrize("center", [True, False])
def test_istft_inverts_stft(oracle, n_fft, hop, L, center):
    """Perfect reconstruction wherever the squared-window sum is positive
    (the division by sum w^2 makes any hop <= n_fft invertible)."""
    x = rnd(2, L)
    w = oracle.hann_window(n_fft)
    for normalized in (False, True):
        y = oracle.istft(oracle.stft(x, n_fft, hop, w, center, normalized), n_fft, hop, w,
                         length=L, center=center, normalized=normalized)
        # covered span: the first sample has w[0] = 0 without centring; the
        # frames end at (T - 1) hop + n_fft (minus the centre padding), and
        # the rest of `length` is zero-padded, as torch.istft does
        lo = 0 if center else 1
        T = (L + (n_fft if center else 0) - n_fft) // hop + 1
        hi = min(L, (T - 1) * hop + n_fft - (n_fft if center else 1))
        # near the uncentred edges sum w^2 is tiny (w[1]^2 ~ 1e-5 at n_fft 64)
        # and the division magnifies the fp32 rounding of the spectrum: compare
        # where sum w^2 > 1e-2
        ws = np.zeros(L + n_fft)
        pad = n_fft // 2 if center else 0
        for t in range(T):
            ws[t * hop:t * hop + n_fft] += w.astype(np.float64) ** 2
        ok = np.nonzero(ws[pad:pad + L] > 1e-2)[0]
        ok = ok[(ok >= lo) & (ok < hi)]
        assert len(ok) > 0.9 * (hi - lo)
        assert rel_err(y[:, ok], x[:, ok]) < 1e-6
        tail = hi if center else hi + 1
        assert np.all(y[:, tail:] == 0)


def test_istft_ignores_dc_and_nyquist_imaginary_parts_and_pads(oracle):
    n_fft, hop = 32, 8
    spec = rnd(1, n_fft // 2 + 1, 6, 2)
    w = oracle.hann_window(n_fft)
    a = oracle.istft(spec, n_fft, hop, w)
    s2 = spec.copy()
    s2[:, 0, :, 1] = 5.0
    s2[:, -1, :, 1] = -3.0
    np.testing.assert_array_equal(oracle.istft(s2, n_fft, hop, w), a)
    longer = oracle.istft(spec, n_fft, hop, w, length=a.shape[1] + 7)
    np.testing.assert_array_equal(longer[:, :a.shape[1]], a)
    assert np.all(longer[:, a.shape[1]:] == 0)
    np.testing.assert_array_equal(oracle.istft(spec, n_fft, hop, w, length=10), a[:, :10])
    # float64 irfft restatement of one frame's contribution
    X = spec[0, :, :, 0].astype(np.float64) + 1j * spec[0, :, :, 1]
    X[0].imag = 0
    X[-1].imag = 0
    fr = np.fft.irfft(X.T, n=n_fft, axis=-1) * w                      # [T, n_fft]
    full = np.zeros(n_fft + 5 * hop)
    ws = np.zeros_like(full)
    for t in range(6):
        full[t * hop:t * hop + n_fft] += fr[t]
        ws[t * hop:t * hop + n_fft] += w.astype(np.float64) ** 2
    full = np.where(ws > 1e-8, full / np.where(ws > 1e-8, ws, 1), full)
    assert rel_err(a[0], full[n_fft // 2:-(n_fft // 2)]) < 1e-6


# ------------------------------------------------- model composition and driver
SMALL_BSR = {"model_type": "bs_roformer", "dim": 128, "depth": 1, "heads": 2, "dim_head": 64,
             "stereo": True, "num_stems": 2, "mask_estimator_depth": 2, "mlp_expansion_factor": 4,
             "zero_dc": False, "stft_n_fft": 256, "stft_hop_length": 64, "stft_win_length": 256,
             "freqs_per_bands": [4] * 8 + [8] * 8 + [16] * 2 + [1], "chunk_size": 4096,
             "num_overlap": 2, "sample_rate": 44100}


def test_process_chunked_identity_model_returns_input(oracle):
    """With a model that returns its input, the fades and the weight
    normalisation cancel: the driver returns the track itself (border
    reflect padding, the reflect / zero-padded last chunk and batching
    included)."""
    for S in (10000, 4096 * 3 + 17, 5000):
        x = rnd(2, S)
        y = oracle.process_chunked(x, 4096, 2048, 2, lambda b: b)
        np.testing.assert_allclose(y, x, rtol=1e-6, atol=1e-6)


def test_bsroformer_forward_unit_mask_returns_input(oracle):
    """A checkpoint whose mask estimators output 1 + 0i leaves the STFT
    untouched: the forward is istft(stft(x)) = x (zero_dc off), which pins
    the layout hand-offs of the composition (gather, merge, stereo split)."""
    import csm_file
    w = csm_file.bsr_checkpoint(SMALL_BSR, seed=1, unit_mask=True)
    x = rnd(1, 2, 64 * 40)
    y = oracle.bsroformer_forward(SMALL_BSR, w, x)
    assert y.shape == (1, 2, 2, 64 * 40)
    for s in range(2):
        assert rel_err(y[0, s], x[0]) < 1e-5


def _htk_triangles_f64(sr, n_fft, n_mels, fmin=0.0, fmax=0.0):
    """Textbook HTK-mel triangles in float64, written as the clipped minimum
    of the two slopes (a different formulation from the piecewise one)."""
    fmax = fmax if fmax > 0 else sr / 2
    hz2mel = lambda f: 2595.0 * np.log10(1.0 + f / 700.0)
    mel2hz = lambda m: 700.0 * (10.0 ** (m / 2595.0) - 1.0)
    e = mel2hz(np.linspace(hz2mel(fmin), hz2mel(fmax), n_mels + 2))
    f = sr * np.arange(n_fft // 2 + 1) / n_fft
    up = (f[None, :] - e[:-2, None]) / (e[1:-1, None] - e[:-2, None])
    down = (e[2:, None] - f[None, :]) / (e[2:, None] - e[1:-1, None])
    return np.maximum(0.0, np.minimum(up, down)), e, f


MEL_CASES = [(44100, 2048, 60, 0.0, 0.0), (44100, 256, 16, 0.0, 0.0),
             (48000, 1024, 40, 0.0, 0.0), (16000, 512, 10, 50.0, 7000.0)]


@pytest.mark.parametrize("sr,n_fft,n_mels,fmin,fmax", MEL_CASES)
def test_mel_filterbank_matches_float64_triangles(oracle, sr, n_fft, n_mels, fmin, fmax):
    fb = oracle.mel_filterbank(sr, n_fft, n_mels, fmin, fmax)
    ref, e, f = _htk_triangles_f64(sr, n_fft, n_mels, fmin, fmax)
    assert fb.shape == ref.shape
    np.testing.assert_allclose(fb, ref, atol=2e-4)
    # Membership agrees wherever the bin is not within 0.05 Hz of an edge
    # (where float and float64 may round to opposite sides).
    tie = (np.abs(f[None, :] - e[:-2, None]) < 0.05) | (np.abs(f[None, :] - e[2:, None]) < 0.05)
    assert np.array_equal((fb > 0)[~tie], (ref > 0)[~tie])


@pytest.mark.parametrize("sr,n_fft,n_mels,fmin,fmax", MEL_CASES)
def test_mel_filterbank_partition_of_unity(oracle, sr, n_fft, n_mels, fmin, fmax):
    """Adjacent HTK triangles share their edges, so between the first and
    the last centre the filters sum to 1 on every bin (an index slip in the
    edges breaks this)."""
    fb = oracle.mel_filterbank(sr, n_fft, n_mels, fmin, fmax)
    _, e, f = _htk_triangles_f64(sr, n_fft, n_mels, fmin, fmax)
    inner = (f >= e[1] + 1e-3) & (f <= e[n_mels] - 1e-3)
    assert inner.sum() > 0
    np.testing.assert_allclose(fb.sum(axis=0)[inner], 1.0, atol=2e-5)
    assert fb.min() >= 0.0 and fb.max() <= 1.0 + 1e-6


def test_mel_filterbank_single_band_closed_form(oracle):
    """n_mels 1: one triangle from fmin to fmax peaking at the mel midpoint."""
    sr, n_fft = 22050, 64
    fb = oracle.mel_filterbank(sr, n_fft, 1)[0]
    mid = 700.0 * (10.0 ** ((2595.0 * np.log10(1.0 + sr / 2 / 700.0)) / 2 / 2595.0) - 1.0)
    f = sr * np.arange(n_fft // 2 + 1) / n_fft
    ref = np.where(f <= mid, f / mid, (sr / 2 - f) / (sr / 2 - mid))
    np.testing.assert_allclose(fb, ref, atol=1e-5)


@pytest.mark.parametrize("sr,n_fft,nb,ch", [(44100, 2048, 60, 2), (44100, 256, 16, 2),
                                            (44100, 2048, 60, 1)])
def test_mel_bands_cover_every_bin_and_interleave(oracle, sr, n_fft, nb, ch):
    fidx, counts = oracle.mel_bands(sr, n_fft, nb, ch)
    F = n_fft // 2 + 1
    assert len(counts) == nb and counts.min() >= 1 and len(fidx) == counts.sum() * ch
    mono = fidx[::ch] // ch
    for s in range(ch):
        assert np.array_equal(fidx[s::ch], mono * ch + s)
    assert np.array_equal(np.unique(mono), np.arange(F))   # every bin in some band
    off = np.concatenate([[0], np.cumsum(counts)])
    first = mono[off[:-1]]
    last = mono[off[1:] - 1]
    assert first[0] == 0 and last[-1] == F - 1               # the two forced corners
    assert np.all(np.diff(first) >= 0) and np.all(np.diff(last) >= 0)
    for b in range(nb):                                      # contiguous runs of bins
        seg = mono[off[b]:off[b + 1]]
        assert np.array_equal(seg, np.arange(seg[0], seg[0] + len(seg)))


SMALL_MBR = {"model_type": "mel_band_roformer", "dim": 64, "depth": 1, "heads": 2,
             "dim_head": 32, "stereo": True, "num_stems": 2, "num_bands": 16,
             "mask_estimator_depth": 2, "mlp_expansion_factor": 4, "zero_dc": False,
             "stft_n_fft": 256, "stft_hop_length": 64, "stft_win_length": 256,
             "sample_rate": 44100}


@pytest.mark.parametrize("precomputed", [False, True])
def test_melbandroformer_forward_unit_mask_returns_input(oracle, precomputed):
    """Unit masks on overlapping bands: the scatter-mean is 1 on every bin,
    so the forward is istft(stft(x)) = x."""
    import csm_file
    if precomputed:
        fidx, counts = csm_file.overlapping_bands(129, 2, 16)
        w = csm_file.mbr_checkpoint(SMALL_MBR, counts, seed=2, unit_mask=True,
                                    precomputed=(fidx, counts))
    else:
        _, counts = oracle.mel_bands(44100, 256, 16, 2)
        w = csm_file.mbr_checkpoint(SMALL_MBR, counts, seed=2, unit_mask=True)
    x = rnd(1, 2, 64 * 40)
    y = oracle.melbandroformer_forward(SMALL_MBR, w, x)
    assert y.shape == (1, 2, 2, 64 * 40)
    for s in range(2):
        assert rel_err(y[0, s], x[0]) < 1e-5


def test_process_chunked_crossfade_closed_form(oracle):
    """A model that outputs its chunk's first sample everywhere exposes the
    windows: on a ramp input, the stitched track between two chunk starts
    is the weighted mean of two constants, so the linear fades (chunk / 10
    samples, i / (fade - 1)), the step, the border reflect padding and the
    untouched first chunk start follow in closed form (inference_app.cpp:
    100-324).  The identity-model check cannot see any of these."""
    C, step, S = 1000, 500, 5000
    fade, border = C // 10, C - step
    x = np.arange(S, dtype=np.float32)[None]
    y = oracle.process_chunked(x, C, step, 3, lambda b: np.repeat(b[:, :, :1], C, axis=2))[0]
    assert y.shape == (S,)
    r = lambda i: i / (fade - 1)
    # Chunk starts (padded coordinates) st = 1500 and 2000 carry the values
    # st - border = 1000 and 1500; they share padded positions [2000, 2500).
    a, b = 1000.0, 1500.0
    for p in range(2000, 2500):
        t = p - border
        if p < 2000 + fade:          # fade-in of the later chunk
            w = r(p - 2000)
            want = (a + w * b) / (1 + w)
        elif p >= 2500 - fade:       # fade-out of the earlier chunk
            w = 1 - r(p - (2500 - fade))
            want = (w * a + b) / (w + 1)
        else:
            want = (a + b) / 2
        assert abs(y[t] - want) <= 1e-3 * abs(want), (t, y[t], want)
    # Track start: padded chunk 0 holds the reflected x[border] = 500 with
    # no fade-in; the chunk at st = 500 holds x[0] = 0 and fades in.
    for t in range(fade):
        w = r(t)
        want = 500.0 / (1 + w)
        assert abs(y[t] - want) <= 1e-3 * want, (t, y[t], want)


# ------------------------------------- depth-loop switches and forward chain
def _identity_layer(rng, dim, H, Dh, ff, final_norm=False):
    """A transformer whose attention and feed-forward branches are exactly 0
    (zero out-projection, zero second linear and bias): x -> x, then the
    optional closing norm."""
    w = R.random_layer(rng, dim, H, Dh, ff, final_norm=final_norm)
    w["w_out"][:] = 0.0
    w["w_ff2"][:] = 0.0
    w["b_ff2"][:] = 0.0
    return w


def test_stack_schedule_default_equals_stack(oracle):
    """time/freq depth 1 without skip: the schedule restatement and the C
    stack (pinned above against the torch composition) agree bit for bit."""
    rng = np.random.default_rng(21)
    B, T, Fb, dim, H, Dh, ff, depth = 2, 7, 5, 32, 2, 16, 64, 2
    layers = [oracle.LayerWeights(**R.random_layer(rng, dim, H, Dh, ff, final_norm=(i % 2 == 1)))
              for i in range(2 * depth)]
    fg = (1 + rng.standard_normal(dim) * 0.02).astype(np.float32)
    x = rng.standard_normal((B, T, Fb, dim)).astype(np.float32)
    np.testing.assert_array_equal(oracle.roformer_stack_schedule(x, layers, H, Dh, fg),
                                  oracle.roformer_stack(x, layers, H, Dh, fg))


def test_stack_schedule_skip_connection_closed_form(oracle):
    """Identity transformers with skip_connection: depth d's output is
    y_d = y_(d-1) + sum_(j<d) y_j (model_bs_roformer.cu:482-487 adds every
    stored output, the previous depth's included), so y = x * (1, 2, 5, 13,
    34)[depth - 1].  Values k/16 keep every sum exact in float32.  Storing
    before the adds, or adding only the last output, gives other factors."""
    rng = np.random.default_rng(22)
    B, T, Fb, dim, H, Dh, ff = 1, 5, 3, 32, 2, 16, 64
    x = (rng.integers(-100, 100, (B, T, Fb, dim)) / 16.0).astype(np.float32)
    for depth, factor in ((1, 1), (2, 2), (3, 5), (4, 13), (5, 34)):
        layers = [oracle.LayerWeights(**_identity_layer(rng, dim, H, Dh, ff))
                  for _ in range(2 * depth)]
        y = oracle.roformer_stack_schedule(x, layers, H, Dh, None, 1, 1, True)
        np.testing.assert_array_equal(y, factor * x)
        np.testing.assert_array_equal(
            oracle.roformer_stack_schedule(x, layers, H, Dh, None, 1, 1, False), x)


@pytest.mark.parametrize("mbr", [False, True])
def test_stack_schedule_transformer_depth(oracle, mbr):
    """time/freq_transformer_depth 2 whose second layers are identities equal
    the depth-1 stack of the first layers (the closing MelBandRoformer norm on
    the last layer of each transformer): a loop that runs the layers in
    another order, interleaves the axes or applies the closing norm after
    every layer fails it (RMSNorm with gamma != 1 is not idempotent)."""
    rng = np.random.default_rng(23)
    B, T, Fb, dim, H, Dh, ff, depth = 1, 6, 4, 32, 2, 16, 64, 2
    firsts = [R.random_layer(rng, dim, H, Dh, ff) for _ in range(2 * depth)]
    fgs = [(1 + rng.standard_normal(dim) * 0.3).astype(np.float32) for _ in range(2 * depth)]
    sched, plain = [], []
    for d in range(depth):
        for t in range(2):
            i = 2 * d + t
            a = dict(firsts[i])
            ident = _identity_layer(rng, dim, H, Dh, ff)
            if mbr:
                ident["final_gamma"] = fgs[i]
                plain.append(oracle.LayerWeights(**dict(a, final_gamma=fgs[i])))
            else:
                plain.append(oracle.LayerWeights(**a))
            sched += [oracle.LayerWeights(**a), oracle.LayerWeights(**ident)]
    # per depth: time_depth (2) time layers, then freq_depth (2) freq layers
    order = []
    for d in range(depth):
        order += [sched[4 * d], sched[4 * d + 1], sched[4 * d + 2], sched[4 * d + 3]]
    x = rng.standard_normal((B, T, Fb, dim)).astype(np.float32)
    y = oracle.roformer_stack_schedule(x, order, H, Dh, None, 2, 2, False)
    r = oracle.roformer_stack(x, plain, H, Dh, None)
    assert rel_err(y, r) < 1e-6
    # the list order is per depth time layers then frequency layers: the
    # interleaved order (time, freq, time, freq) runs the frequency weights
    # on the time axis and must give another result
    inter = []
    for d in range(depth):
        inter += [sched[4 * d], sched[4 * d + 2], sched[4 * d + 1], sched[4 * d + 3]]
    assert rel_err(oracle.roformer_stack_schedule(x, inter, H, Dh, None, 2, 2, False), r) > 1e-3


def _np_istft(spec, n_fft, hop, w, length):
    """torch.istft restated with numpy: irfft per frame (the imaginary DC /
    Nyquist parts drop out), window, overlap-add, divide by the summed
    squared window where it exceeds 1e-8, trim the centre padding."""
    X = spec[..., 0].astype(np.float64) + 1j * spec[..., 1]          # [B, F, T]
    fr = np.fft.irfft(X.transpose(0, 2, 1), n=n_fft, axis=-1) * w    # [B, T, n_fft]
    B, T = fr.shape[:2]
    n = n_fft + hop * (T - 1)
    out = np.zeros((B, n))
    ws = np.zeros(n)
    for t in range(T):
        out[:, t * hop:t * hop + n_fft] += fr[:, t]
        ws[t * hop:t * hop + n_fft] += w ** 2
    out = np.where(ws > 1e-8, out / np.where(ws > 1e-8, ws, 1.0), out)
    out = out[:, n_fft // 2:n - n_fft // 2]
    return out if length < 0 else out[:, :length]


def _np_rms(x, gamma, scale):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).sum(-1, keepdims=True) + 1e-12) * gamma * scale


def _np_identity_forward(cfg, w, audio, dims, fidx, norms, L):
    """float64 numpy chain of a Roformer forward whose transformers are
    identities (model_bs_roformer.cu:420-609, model_mel_band_roformer.cu:
    745-1040): STFT, 'b s f t c -> b t (f s) c' and the band bin selection
    fidx (None: every bin in order), per band RMSNorm * sqrt(band width) +
    linear, the RMSNorms `norms` in sequence (what is left of the stack: the
    closing norms, or the final norm), per stem band MLPs of L linears (tanh
    between) and GLU, complex masks averaged over the bands that hold each
    bin, times the STFT, zero DC, stereo split, iSTFT."""
    B, ch, S = audio.shape
    n_fft, hop = cfg["stft_n_fft"], cfg["stft_hop_length"]
    win = np.hanning(n_fft + 1)[:-1]
    spec = _np_stft(audio.reshape(B * ch, S), n_fft, hop, win, True, False)   # [B*ch, F, T, 2]
    F, T = spec.shape[1], spec.shape[2]
    g = spec.reshape(B, ch, F, T, 2).transpose(0, 3, 2, 1, 4).reshape(B, T, F * ch, 2)
    fi = np.arange(F * ch) if fidx is None else np.asarray(fidx)
    x = g[:, :, fi].reshape(B, T, -1)
    off = np.concatenate([[0], np.cumsum(dims)])
    feats = []
    for b, d in enumerate(dims):
        p = f"band_split.to_features.{b}"
        xb = _np_rms(x[..., off[b]:off[b + 1]], w[p + ".0.gamma"], math.sqrt(d))
        feats.append(xb @ w[p + ".1.weight"].T.astype(np.float64) + w[p + ".1.bias"])
    f = np.stack(feats, 2)                                                    # [B, T, nb, dim]
    for gam in norms:
        f = _np_rms(f, gam, math.sqrt(cfg["dim"]))
    cnt = np.bincount(fi, minlength=F * ch).astype(np.float64)
    outs = []
    for s in range(cfg["num_stems"]):
        mk = []
        for b, d in enumerate(dims):
            h = f[:, :, b]
            for i in range(L):
                p = f"mask_estimators.{s}.to_freqs.{b}.0.{2 * i}"
                h = h @ w[p + ".weight"].T.astype(np.float64) + w[p + ".bias"]
                if i < L - 1:
                    h = np.tanh(h)
            mk.append(h[..., :d] / (1.0 + np.exp(-h[..., d:])))
        m = np.concatenate(mk, -1)
        mc = m[..., 0::2] + 1j * m[..., 1::2]                                  # [B, T, n]
        acc = np.zeros((B, T, F * ch), np.complex128)
        np.add.at(acc, (slice(None), slice(None), fi), mc)
        mean = (acc / np.maximum(cnt, 1e-8)).reshape(B, T, F, ch)
        xc = (spec[..., 0] + 1j * spec[..., 1]).reshape(B, ch, F, T)
        o = xc * mean.transpose(0, 3, 2, 1)                                    # [B, ch, F, T]
        if cfg.get("zero_dc", True):
            o[:, :, 0] = 0
        o = np.stack([o.real, o.imag], -1).reshape(B * ch, F, T, 2)
        outs.append(_np_istft(o, n_fft, hop, win, -1).reshape(B, ch, -1))
    return np.stack(outs, 1)                                                   # [B, stems, ch, S']


def _zero_branches(w, depth):
    for d in range(depth):
        for t in range(2):
            p = f"layers.{d}.{t}.layers.0"
            w[p + ".0.to_out.0.weight"][:] = 0.0
            w[p + ".1.net.4.weight"][:] = 0.0
            w[p + ".1.net.4.bias"][:] = 0.0


def test_bsroformer_forward_chain_with_identity_stack(oracle):
    """Zero out-projections and second linears make every transformer the
    identity; the forward then reduces to the float64 numpy chain above, which
    pins the composition's middle (band split -> final norm -> mask MLPs ->
    merge).  The same chain without the final norm (a planted bug) must not
    match."""
    import csm_file
    cfg = dict(SMALL_BSR, depth=2, zero_dc=True)
    w = csm_file.bsr_checkpoint(cfg, seed=5)
    _zero_branches(w, cfg["depth"])
    x = rnd(1, 2, 64 * 30)
    y = oracle.bsroformer_forward(cfg, w, x)
    dims = [4 * f for f in cfg["freqs_per_bands"]]
    L = cfg["mask_estimator_depth"]
    r = _np_identity_forward(cfg, w, x, dims, None, [w["final_norm.gamma"]], L)
    assert y.shape == r.shape
    assert rel_err(y, r) < 1e-4
    bug = _np_identity_forward(cfg, w, x, dims, None, [], L)
    assert rel_err(y, bug) > 1e-2


def test_melbandroformer_forward_chain_with_identity_stack(oracle):
    """The MelBandRoformer chain with identity transformers: what remains of
    the stack is the norm closing every transformer, in order (time then
    frequency per depth), on overlapping bands whose masks are averaged per
    bin.  Dropping one closing norm (a planted bug) must not match."""
    import csm_file
    cfg = dict(SMALL_MBR, depth=2, zero_dc=True)
    fidx, counts = csm_file.overlapping_bands(129, 2, 16)
    w = csm_file.mbr_checkpoint(cfg, counts, seed=6, precomputed=(fidx, counts))
    _zero_branches(w, cfg["depth"])
    x = rnd(1, 2, 64 * 30)
    y = oracle.melbandroformer_forward(cfg, w, x)
    dims = [4 * int(c) for c in counts]
    norms = [w[f"layers.{d}.{t}.norm.gamma"] for d in range(2) for t in range(2)]
    L = cfg["mask_estimator_depth"] + 1
    r = _np_identity_forward(cfg, w, x, dims, fidx, norms, L)
    assert y.shape == r.shape
    assert rel_err(y, r) < 1e-4
    bug = _np_identity_forward(cfg, w, x, dims, fidx, norms[:-1], L)
    assert rel_err(y, bug) > 1e-2
