"""Writes the reference's converted-checkpoint container (.csm, the format
src/weights.cu:412-508 reads): "CSM\\0", u32 version 1, u32 + config JSON,
u32 tensor count, then per tensor u32 + name, u32 ndim, i64 dims, u32 dtype
(0 f32, 1 f16, 2 i64), raw little-endian data.  Test helper: builds
synthetic BSRoformer and MelBandRoformer checkpoints (random weights of the
reference's names/shapes)."""
from __future__ import annotations

import json
import math
import struct

import numpy as np


def write_csm(path, config: dict, tensors: dict) -> None:
    cfg = json.dumps(config).encode()
    with open(path, "wb") as f:
        f.write(b"CSM\0")
        f.write(struct.pack("<II", 1, len(cfg)))
        f.write(cfg)
        f.write(struct.pack("<I", len(tensors)))
        for name, a in tensors.items():
            a = np.ascontiguousarray(a)
            code = {np.dtype(np.float32): 0, np.dtype(np.float16): 1, np.dtype(np.int64): 2}[a.dtype]
            nb = name.encode()
            f.write(struct.pack("<I", len(nb)) + nb)
            f.write(struct.pack("<I", a.ndim) + struct.pack(f"<{a.ndim}q", *a.shape))
            f.write(struct.pack("<I", code))
            f.write(a.tobytes())


def _roformer_weights(cfg: dict, band_bins, seed: int, unit_mask: bool, L: int,
                      per_norm: bool, final_norm: bool) -> dict:
    """Random weights under the names both Roformers read
    (model_bs_roformer.cu:111-183, model_mel_band_roformer.cu:380-470).
    unit_mask: every mask estimator outputs mask 1 + 0i (last layer weights
    0; value bias (1, 0), gate bias 40)."""
    rng = np.random.default_rng(seed)
    ch = 2 if cfg.get("stereo", True) else 1
    dim, depth, heads, dh = cfg["dim"], cfg["depth"], cfg["heads"], cfg.get("dim_head", 64)
    ff = dim * cfg.get("mlp_expansion_factor", 4)
    inner = heads * dh

    def lin(n, k):
        return (rng.standard_normal((n, k)) / math.sqrt(k)).astype(np.float32)

    def vec(n, s=0.02, m=0.0):
        return (m + s * rng.standard_normal(n)).astype(np.float32)

    w = {}
    for b, f in enumerate(band_bins):
        d = 2 * f * ch
        p = f"band_split.to_features.{b}"
        w[p + ".0.gamma"] = vec(d, m=1.0)
        w[p + ".1.weight"] = lin(dim, d)
        w[p + ".1.bias"] = vec(dim)
    td, fd = cfg.get("time_transformer_depth", 1), cfg.get("freq_transformer_depth", 1)
    for d_ in range(depth):
        for t, li in [(0, i) for i in range(td)] + [(1, i) for i in range(fd)]:
            p = f"layers.{d_}.{t}.layers.{li}"
            w[p + ".0.norm.gamma"] = vec(dim, m=1.0)
            w[p + ".0.to_qkv.weight"] = lin(3 * inner, dim)
            w[p + ".0.to_gates.weight"] = lin(heads, dim)
            w[p + ".0.to_gates.bias"] = vec(heads)
            w[p + ".0.to_out.0.weight"] = lin(dim, inner) * 0.5
            w[p + ".1.net.0.gamma"] = vec(dim, m=1.0)
            w[p + ".1.net.1.weight"] = lin(ff, dim)
            w[p + ".1.net.1.bias"] = vec(ff)
            w[p + ".1.net.4.weight"] = lin(dim, ff) * 0.5
            w[p + ".1.net.4.bias"] = vec(dim)
            if per_norm and li == (td if t == 0 else fd) - 1:
                w[f"layers.{d_}.{t}.norm.gamma"] = vec(dim, 0.1, m=1.0)
    if final_norm:
        w["final_norm.gamma"] = vec(dim, m=1.0)
    hid = dim * cfg.get("mlp_expansion_factor", 4)
    for s in range(cfg.get("num_stems", 1)):
        for b, f in enumerate(band_bins):
            d = 2 * f * ch
            K = dim
            for i in range(L):
                N = 2 * d if i == L - 1 else hid
                p = f"mask_estimators.{s}.to_freqs.{b}.0.{2 * i}"
                w[p + ".weight"] = lin(N, K)
                w[p + ".bias"] = vec(N)
                if unit_mask and i == L - 1:
                    w[p + ".weight"][:] = 0.0
                    bias = np.zeros(N, np.float32)
                    bias[0:d:2] = 1.0       # value half: real parts 1, imaginary 0
                    bias[d:] = 40.0         # gate half: sigmoid -> 1
                    w[p + ".bias"] = bias
                K = N
    return w


def overlapping_bands(F: int, ch: int, nb: int, width: int = 12, stride: int = 8):
    """nb bands of `width` bins every `stride` bins, the last one running to
    bin F - 1 (so each bin sits in one or two bands): channel-interleaved
    freq_indices and bins per band, as int64."""
    bands = [np.arange(b * stride, F if b == nb - 1 else min(b * stride + width, F))
             for b in range(nb)]
    mono = np.concatenate(bands)
    fidx = (mono[:, None] * ch + np.arange(ch)[None, :]).reshape(-1)
    return fidx.astype(np.int64), np.array([len(b) for b in bands], np.int64)


def bsr_checkpoint(cfg: dict, seed: int = 0, unit_mask: bool = False) -> dict:
    """Random BSRoformer weights (mask_estimator_depth linears per band MLP,
    global final norm)."""
    return _roformer_weights(cfg, cfg["freqs_per_bands"], seed, unit_mask,
                             cfg.get("mask_estimator_depth", 1), False, True)


def mbr_checkpoint(cfg: dict, band_bins, seed: int = 0, unit_mask: bool = False,
                   precomputed=None) -> dict:
    """Random MelBandRoformer weights for bands of band_bins bins each
    (mask_estimator_depth + 1 linears per band MLP, a norm closing every
    transformer, no final norm).  precomputed = (freq_indices with the
    channels interleaved, bins per band): stored as the converter's
    __precomputed__ int64 tensors (tools/convert_weights.py:262-316)."""
    w = _roformer_weights(cfg, band_bins, seed, unit_mask,
                          cfg.get("mask_estimator_depth", 2) + 1, True, False)
    if precomputed is not None:
        fidx, counts = (np.asarray(a, np.int64) for a in precomputed)
        ch = 2 if cfg.get("stereo", True) else 1
        F = cfg["stft_n_fft"] // 2 + 1
        w["__precomputed__.freq_indices"] = fidx
        w["__precomputed__.num_freqs_per_band"] = counts
        w["__precomputed__.num_bands_per_freq"] = np.bincount(fidx[::ch] // ch,
                                                              minlength=F).astype(np.int64)
    return w
