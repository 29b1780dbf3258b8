"""STFT / iSTFT (hand-written FFT) against the CPU oracle (float64 FFT,
pinned against numpy.fft in tests/test_oracle.py), at the Roformers' setting
(n_fft 2048, hop 441, Hann, 8 s stereo at 44.1 kHz) and small edge cases.
fp32 path: tolerance 1e-5 normwise (the FFT's own rounding is ~1e-7 per
pass, log2 n passes)."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

TOL = 1e-5


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def test_hann_window(msst, oracle, cuda):
    for n in (1, 16, 2048, 4096):
        np.testing.assert_allclose(host(msst.hann_window(n)), oracle.hann_window(n), atol=2e-7)


CASES = [(2, 352800, 2048, 441), (1, 5000, 2048, 441), (3, 1000, 256, 64), (2, 300, 64, 17),
         (1, 4096, 4096, 1024), (1, 700, 512, 512), (2, 100, 16, 3), (1, 20000, 4096, 2205)]


@pytest.mark.parametrize("B,L,n_fft,hop", CASES)
@pytest.mark.parametrize("center", [True, False])
@pytest.mark.parametrize("normalized", [False, True])
def test_stft(msst, oracle, cuda, B, L, n_fft, hop, center, normalized):
    if center and L <= n_fft // 2:
        pytest.skip("reflect padding needs L > n_fft / 2")
    if not center and L < n_fft:
        pytest.skip("no frame without centring")
    rng = np.random.default_rng(L + n_fft)
    x = rng.standard_normal((B, L)).astype(np.float32)
    w = oracle.hann_window(n_fft)
    y = host(msst.stft(dev(x), n_fft, hop, dev(w), center, normalized))
    r = oracle.stft(x, n_fft, hop, w, center, normalized)
    assert y.shape == r.shape
    assert rel_err(y, r) < TOL


@pytest.mark.parametrize("B,L,n_fft,hop", CASES)
@pytest.mark.parametrize("center", [True, False])
@pytest.mark.parametrize("length", ["full", "short", "long"])
def test_istft(msst, oracle, cuda, B, L, n_fft, hop, center, length):
    rng = np.random.default_rng(L + 3 * n_fft)
    T = max(2, L // hop)
    spec = rng.standard_normal((B, n_fft // 2 + 1, T, 2)).astype(np.float32)
    w = oracle.hann_window(n_fft)
    full = n_fft + (T - 1) * hop - (n_fft if center else 0)
    ln = {"full": -1, "short": max(1, full // 2), "long": full + 777}[length]
    if full < 1:
        pytest.skip("nothing left after trimming")
    for normalized in (False, True):
        y = host(msst.istft(dev(spec), n_fft, hop, dev(w), ln, center, normalized))
        r = oracle.istft(spec, n_fft, hop, w, ln, center, normalized)
        assert y.shape == r.shape
        assert rel_err(y, r) < TOL


def test_round_trip_8s_stereo(msst, cuda):
    """stft -> istft on the Roformers' setting reconstructs the signal (the
    division by sum w^2 makes it exact up to rounding), on the GPU alone."""
    x = torch.randn(2, 352800, device="cuda")
    w = msst.hann_window(2048)
    s = msst.stft(x, 2048, 441, w)
    assert s.shape == (2, 1025, 801, 2)
    y = msst.istft(s, 2048, 441, w, length=352800)
    n = 352800 - 352800 % 441   # frames cover the first 800 hops + n_fft / 2
    assert rel_err(host(y)[:, :n], host(x)[:, :n]) < 2e-6


def test_rejects_unsupported_sizes(msst, cuda):
    x = torch.zeros(1, 10000, device="cuda")
    with pytest.raises(RuntimeError, match="power of two"):
        msst.stft(x, 8192, 441, torch.ones(8192, device="cuda"))
    with pytest.raises(RuntimeError):
        msst.stft(x[:, :100], 2048, 441, torch.ones(2048, device="cuda"))  # too short to reflect
