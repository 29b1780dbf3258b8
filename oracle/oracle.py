"""ctypes wrapper of the CPU oracle (oracle/_build/libmsst_oracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the timed
CPU baseline of bench.py.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module; the product never does.

All arrays are numpy float32, C-contiguous.  Functions return new arrays and
never modify their inputs, except where the name says `_inplace`.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass, fields

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libmsst_oracle.so")

ACT = {"none": 0, "gelu": 1, "sigmoid": 2, "silu": 3, "tanh": 4}

_lib = None


def build() -> None:
    """Compile the oracle with its Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_fp = ctypes.POINTER(ctypes.c_float)
_i64 = ctypes.c_int64


class LayerWeightsC(ctypes.Structure):
    _fields_ = [(n, _fp) for n in (
        "attn_gamma", "w_qkv", "w_gate", "b_gate", "w_out", "ff_gamma",
        "w_ff1", "b_ff1", "w_ff2", "b_ff2", "final_gamma")]


def _declare(l: ctypes.CDLL) -> None:
    l.orc_num_threads.restype = ctypes.c_int
    l.orc_set_num_threads.argtypes = [ctypes.c_int]
    l.orc_linear.argtypes = [_fp, _fp, _fp, _fp, _fp, _i64, _i64, _i64, ctypes.c_int]
    l.orc_activation.argtypes = [_fp, _fp, _i64, ctypes.c_int]
    l.orc_rms_norm.argtypes = [_fp, _fp, ctypes.c_float, _fp, _i64, _i64]
    l.orc_rope_table.argtypes = [ctypes.c_int, ctypes.c_int, _fp, _fp]
    l.orc_rope_apply.argtypes = [_fp, _fp, _fp, _fp, _i64, _i64, _i64, _i64]
    l.orc_attention.argtypes = [_fp, _fp, _fp, _fp, _i64, _i64, _i64, _i64, _i64,
                                ctypes.c_float]
    l.orc_split_qkv.argtypes = [_fp, _fp, _fp, _fp, _i64, _i64, _i64, _i64]
    l.orc_gate_merge.argtypes = [_fp, _fp, _fp, _i64, _i64, _i64, _i64]
    l.orc_transformer.argtypes = [_fp, _i64, _i64, _i64, _i64, _i64, _i64,
                                  ctypes.POINTER(LayerWeightsC), _fp, _fp]
    l.orc_roformer_stack.argtypes = [_fp, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _i64, ctypes.POINTER(LayerWeightsC), _fp]
    _ip = ctypes.POINTER(ctypes.c_int)
    l.orc_glu.argtypes = [_fp, _fp, _i64, _i64]
    l.orc_band_split.argtypes = [_fp, _i64, _ip, ctypes.c_int, _fp, _fp, _fp, _fp, _i64]
    l.orc_mask_estimator.argtypes = [_fp, _i64, _ip, ctypes.c_int, _i64, _i64, ctypes.c_int,
                                     _fp, _fp, _fp]
    l.orc_band_gather.argtypes = [_fp, _i64, _i64, _i64, _i64, _ip, _i64, _fp]
    l.orc_stft.argtypes = [_fp, _i64, _i64, ctypes.c_int, ctypes.c_int, _fp, ctypes.c_int,
                           ctypes.c_int, _fp]
    l.orc_istft.argtypes = [_fp, _i64, _i64, ctypes.c_int, ctypes.c_int, _fp, _i64, ctypes.c_int,
                            ctypes.c_int, _fp]
    l.orc_hann_window.argtypes = [_fp, ctypes.c_int]
    l.orc_mel_filterbank.argtypes = [_fp, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_float, ctypes.c_float]
    l.orc_mask_merge.argtypes = [_fp, _i64, _fp, _i64, _i64, _i64, _i64, _ip, _i64, ctypes.c_int,
                                 _fp]


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _p(a):
    if a is None:
        return None
    return a.ctypes.data_as(_fp)


def num_threads() -> int:
    return lib().orc_num_threads()


def set_num_threads(n: int) -> None:
    lib().orc_set_num_threads(n)


def linear(x, w, b=None, act="none", residual=None) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    K = x.shape[-1]
    N, Kw = w.shape
    assert Kw == K
    M = x.size // K
    b = None if b is None else _f32(b)
    r = None if residual is None else _f32(residual).reshape(M, N)
    out = np.empty(x.shape[:-1] + (N,), np.float32)
    lib().orc_linear(_p(x), _p(w), _p(b), _p(r), _p(out), M, K, N, ACT[act])
    return out


def activation(x, act) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_activation(_p(x), _p(out), x.size, ACT[act])
    return out


def rms_norm(x, gamma, scale) -> np.ndarray:
    x, g = _f32(x), _f32(gamma)
    D = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_rms_norm(_p(x), _p(g), float(scale), _p(out), x.size // D, D)
    return out


def rope_table(n: int, dh: int):
    c = np.empty((n, dh // 2), np.float32)
    s = np.empty((n, dh // 2), np.float32)
    lib().orc_rope_table(n, dh, _p(c), _p(s))
    return c, s


def rope_apply(q, k, cos_t, sin_t):
    q = _f32(q).copy()
    k = _f32(k).copy()
    B, H, N, D = q.shape
    lib().orc_rope_apply(_p(q), _p(k), _p(_f32(cos_t)), _p(_f32(sin_t)), B, H, N, D)
    return q, k


def attention(q, k, v, scale=None) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    B, H, N, D = q.shape
    Nk = k.shape[2]
    if scale is None or scale == 0.0:
        scale = 1.0 / np.sqrt(np.float32(D))
    out = np.empty_like(q)
    lib().orc_attention(_p(q), _p(k), _p(v), _p(out), B, H, N, Nk, D, float(scale))
    return out


def split_qkv(qkv, H, D):
    qkv = _f32(qkv)
    B, N, _ = qkv.shape
    q = np.empty((B, H, N, D), np.float32)
    k = np.empty_like(q)
    v = np.empty_like(q)
    lib().orc_split_qkv(_p(qkv), _p(q), _p(k), _p(v), B, N, H, D)
    return q, k, v


def gate_merge(o, gates) -> np.ndarray:
    o, g = _f32(o), _f32(gates)
    B, H, N, D = o.shape
    out = np.empty((B, N, H * D), np.float32)
    lib().orc_gate_merge(_p(o), _p(g), _p(out), B, H, N, D)
    return out


@dataclass
class LayerWeights:
    """fp32 weights of one transformer, nn.Linear layout ([out, in])."""
    attn_gamma: np.ndarray
    w_qkv: np.ndarray
    w_gate: np.ndarray
    b_gate: np.ndarray
    w_out: np.ndarray
    ff_gamma: np.ndarray
    w_ff1: np.ndarray
    b_ff1: np.ndarray
    w_ff2: np.ndarray
    b_ff2: np.ndarray
    final_gamma: np.ndarray | None = None

    def to_c(self) -> LayerWeightsC:
        kw = {}
        for f in fields(self):
            a = getattr(self, f.name)
            if a is not None:
                a = _f32(a)
                setattr(self, f.name, a)  # keep the contiguous copy alive
            kw[f.name] = _p(a)
        return LayerWeightsC(**kw)


def transformer(x, w: LayerWeights, cos_t, sin_t, heads: int, dim_head: int) -> np.ndarray:
    x = _f32(x).copy()
    B, N, dim = x.shape
    ff = w.w_ff1.shape[0]
    wc = w.to_c()
    cos_t, sin_t = _f32(cos_t), _f32(sin_t)
    lib().orc_transformer(_p(x), B, N, dim, heads, dim_head, ff, ctypes.byref(wc),
                          _p(cos_t), _p(sin_t))
    return x


def roformer_stack(x, layers, heads: int, dim_head: int, final_gamma=None) -> np.ndarray:
    """x: [B, T, F, dim]; layers: [time0, freq0, time1, freq1, ...]."""
    x = _f32(x).copy()
    B, T, F, dim = x.shape
    assert len(layers) % 2 == 0
    ff = layers[0].w_ff1.shape[0]
    arr = (LayerWeightsC * len(layers))(*[lw.to_c() for lw in layers])
    fg = None if final_gamma is None else _f32(final_gamma)
    lib().orc_roformer_stack(_p(x), B, T, F, dim, heads, dim_head, ff, len(layers) // 2,
                             arr, _p(fg))
    return x


def roformer_stack_schedule(x, layers, heads: int, dim_head: int, final_gamma=None,
                            time_depth: int = 1, freq_depth: int = 1,
                            skip_connection: bool = False) -> np.ndarray:
    """The depth loop of model_bs_roformer.cu:477-539 with its configuration
    switches: per depth, skip_connection adds every stored earlier depth
    output, one at a time (:482-487); then the time transformer on
    [B*F, T, dim] (:488-505) as time_depth layers in sequence (the
    apply_transformer loop, :319-327), the frequency transformer on
    [B*T, F, dim] as freq_depth layers (:507-530); the depth output is stored
    (:531-535).  layers: per depth, time_depth then freq_depth entries (a
    MelBandRoformer transformer's closing norm on its last layer).
    final_gamma: BSRoformer's final norm (:538-539)."""
    x = _f32(x).copy()
    B, T, F, dim = x.shape
    per = time_depth + freq_depth
    assert len(layers) % per == 0
    depth = len(layers) // per
    tc, ts = rope_table(T, dim_head)
    fc, fs = rope_table(F, dim_head)
    store = []
    for d in range(depth):
        if skip_connection:
            for j in range(d):
                x = x + store[j]
        xt = np.ascontiguousarray(x.transpose(0, 2, 1, 3)).reshape(B * F, T, dim)
        for i in range(time_depth):
            xt = transformer(xt, layers[d * per + i], tc, ts, heads, dim_head)
        x = np.ascontiguousarray(xt.reshape(B, F, T, dim).transpose(0, 2, 1, 3))
        xf = x.reshape(B * T, F, dim)
        for i in range(freq_depth):
            xf = transformer(xf, layers[d * per + time_depth + i], fc, fs, heads, dim_head)
        x = xf.reshape(B, T, F, dim)
        if skip_connection:
            store.append(x.copy())
    if final_gamma is not None:
        x = rms_norm(x, final_gamma, float(np.sqrt(dim)))
    return x


def glu(x) -> np.ndarray:
    """x [..., 2n] -> x[..., :n] * sigmoid(x[..., n:])."""
    x = _f32(x)
    n = x.shape[-1] // 2
    out = np.empty(x.shape[:-1] + (n,), np.float32)
    lib().orc_glu(_p(x), _p(out), x.size // (2 * n), n)
    return out


def _dims(dims):
    d = np.ascontiguousarray(dims, dtype=np.int32)
    return d, d.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def band_split(x, dims, gammas, ws, biases) -> np.ndarray:
    """x [rows, sum(dims)]; per band b: gammas[b] [dims[b]], ws[b] [dim, dims[b]],
    biases[b] [dim].  Returns [rows, nb, dim]."""
    x = _f32(x)
    rows = x.shape[0]
    nb = len(dims)
    dim = ws[0].shape[0]
    g = _f32(np.concatenate([np.ravel(a) for a in gammas]))
    w = _f32(np.concatenate([np.ravel(a) for a in ws]))
    b = _f32(np.concatenate([np.ravel(a) for a in biases]))
    d, dp = _dims(dims)
    out = np.empty((rows, nb, dim), np.float32)
    lib().orc_band_split(_p(x), rows, dp, nb, _p(g), _p(w), _p(b), _p(out), dim)
    return out


def mask_estimator(x, dims, ws, biases) -> np.ndarray:
    """x [rows, nb, dim]; ws[b][l] / biases[b][l]: the L linears of band b's
    MLP (tanh between, GLU after).  Returns [rows, sum(dims)]."""
    x = _f32(x)
    rows, nb, dim = x.shape
    L = len(ws[0])
    hid = ws[0][0].shape[0] if L > 1 else 0
    w = _f32(np.concatenate([np.ravel(a) for band in ws for a in band]))
    b = _f32(np.concatenate([np.ravel(a) for band in biases for a in band]))
    d, dp = _dims(dims)
    out = np.empty((rows, int(d.sum())), np.float32)
    lib().orc_mask_estimator(_p(x), rows, dp, nb, dim, hid, L, _p(w), _p(b), _p(out))
    return out


def _fidx(fidx):
    if fidx is None:
        return None, None
    f = np.ascontiguousarray(fidx, dtype=np.int32)
    return f, f.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def band_gather(stft, batch, fidx=None) -> np.ndarray:
    """stft [batch*ch, F, T, 2] -> [batch, T, 2n] (n = len(fidx) or F*ch)."""
    stft = _f32(stft)
    BC, F, T, _ = stft.shape
    ch = BC // batch
    f, fp = _fidx(fidx)
    n = len(f) if f is not None else F * ch
    out = np.empty((batch, T, 2 * n), np.float32)
    lib().orc_band_gather(_p(stft), batch, ch, F, T, fp, n, _p(out))
    return out


def mask_merge(masks, stft, batch, fidx=None, zero_dc=True) -> np.ndarray:
    """masks [stems, batch, T, 2n], stft [batch*ch, F, T, 2] -> [batch*stems*ch, F, T, 2]."""
    masks, stft = _f32(masks), _f32(stft)
    stems = masks.shape[0]
    BC, F, T, _ = stft.shape
    ch = BC // batch
    f, fp = _fidx(fidx)
    n = masks.shape[-1] // 2
    out = np.empty((batch * stems * ch, F, T, 2), np.float32)
    lib().orc_mask_merge(_p(masks), stems, _p(stft), batch, ch, F, T, fp, n, int(zero_dc),
                         _p(out))
    return out


def hann_window(size: int) -> np.ndarray:
    out = np.empty(size, np.float32)
    lib().orc_hann_window(_p(out), size)
    return out


def stft(signal, n_fft, hop, window, center=True, normalized=False) -> np.ndarray:
    """signal [B, L] -> [B, n_fft/2 + 1, T, 2]."""
    x = _f32(signal)
    B, L = x.shape
    w = _f32(window)
    T = (L + (n_fft if center else 0) - n_fft) // hop + 1
    out = np.empty((B, n_fft // 2 + 1, T, 2), np.float32)
    lib().orc_stft(_p(x), B, L, n_fft, hop, _p(w), int(center), int(normalized), _p(out))
    return out


def istft(spec, n_fft, hop, window, length=-1, center=True, normalized=False) -> np.ndarray:
    """spec [B, n_fft/2 + 1, T, 2] -> [B, out_len]."""
    s = _f32(spec)
    B, F, T, _ = s.shape
    w = _f32(window)
    out_len = length if length > 0 else n_fft + (T - 1) * hop - (n_fft if center else 0)
    out = np.empty((B, out_len), np.float32)
    lib().orc_istft(_p(s), B, T, n_fft, hop, _p(w), out_len, int(center), int(normalized),
                    _p(out))
    return out


# ------------------------------------------------------------------ BSRoformer
def mel_filterbank(sr: int, n_fft: int, n_mels: int, fmin: float = 0.0,
                   fmax: float = 0.0) -> np.ndarray:
    """ops::mel_filterbank (ops_misc.cu:469-525): [n_mels, n_fft/2 + 1] fp32."""
    out = np.empty((n_mels, n_fft // 2 + 1), np.float32)
    lib().orc_mel_filterbank(_p(out), sr, n_fft, n_mels, ctypes.c_float(fmin),
                             ctypes.c_float(fmax))
    return out


def mel_bands(sr: int, n_fft: int, num_bands: int, channels: int):
    """MelBandRoformer::compute_mel_bands (model_mel_band_roformer.cu:214-308):
    the filterbank with its two corners forced to 1, thresholded at > 0.
    Returns (freq_indices with the channels interleaved as f * ch + s,
    bins per band)."""
    fb = mel_filterbank(sr, n_fft, num_bands)
    fb[0, 0] = 1.0
    fb[-1, -1] = 1.0
    on = fb > 0
    counts = on.sum(axis=1).astype(np.int64)
    mono = np.concatenate([np.nonzero(on[b])[0] for b in range(num_bands)]).astype(np.int64)
    fidx = (mono[:, None] * channels + np.arange(channels)[None, :]).reshape(-1)
    return fidx, counts


def _roformer_forward(cfg: dict, w: dict, audio, dims, fidx, depth: int, L: int,
                      per_norm: bool, final_gamma) -> np.ndarray:
    audio = _f32(audio)
    B, ch, S = audio.shape
    n_fft, hop = cfg.get("stft_n_fft", 2048), cfg.get("stft_hop_length", 441)
    norm = bool(cfg.get("stft_normalized", False))
    stems = cfg.get("num_stems", 1)
    win = hann_window(n_fft)
    spec = stft(audio.reshape(B * ch, S), n_fft, hop, win, True, norm)      # [B*ch, F, T, 2]
    x = band_gather(spec, B, fidx)
    nb = len(dims)
    feats = band_split(
        x.reshape(-1, x.shape[-1]), dims,
        [w[f"band_split.to_features.{b}.0.gamma"] for b in range(nb)],
        [w[f"band_split.to_features.{b}.1.weight"] for b in range(nb)],
        [w[f"band_split.to_features.{b}.1.bias"] for b in range(nb)])
    T = spec.shape[2]
    feats = feats.reshape(B, T, nb, -1)
    td, fd = cfg.get("time_transformer_depth", 1), cfg.get("freq_transformer_depth", 1)
    skip = bool(cfg.get("skip_connection", False))
    layers = []
    for d in range(depth):
        for t, n in ((0, td), (1, fd)):
            for i in range(n):
                p = f"layers.{d}.{t}.layers.{i}"
                last = per_norm and i == n - 1
                layers.append(LayerWeights(
                    w[p + ".0.norm.gamma"], w[p + ".0.to_qkv.weight"],
                    w[p + ".0.to_gates.weight"], w[p + ".0.to_gates.bias"],
                    w[p + ".0.to_out.0.weight"], w[p + ".1.net.0.gamma"],
                    w[p + ".1.net.1.weight"], w[p + ".1.net.1.bias"], w[p + ".1.net.4.weight"],
                    w[p + ".1.net.4.bias"], w[f"layers.{d}.{t}.norm.gamma"] if last else None))
    if td == 1 and fd == 1 and not skip:
        feats = roformer_stack(feats, layers, cfg.get("heads", 8), cfg.get("dim_head", 64),
                               final_gamma)
    else:
        feats = roformer_stack_schedule(feats, layers, cfg.get("heads", 8),
                                        cfg.get("dim_head", 64), final_gamma, td, fd, skip)
    masks = []
    for s in range(stems):
        ws = [[w[f"mask_estimators.{s}.to_freqs.{b}.0.{2 * i}.weight"] for i in range(L)]
              for b in range(nb)]
        bs = [[w[f"mask_estimators.{s}.to_freqs.{b}.0.{2 * i}.bias"] for i in range(L)]
              for b in range(nb)]
        masks.append(mask_estimator(feats.reshape(B * T, nb, -1), dims, ws, bs).reshape(B, T, -1))
    merged = mask_merge(np.stack(masks), spec, B, fidx, bool(cfg.get("zero_dc", True)))
    length = S if cfg.get("match_input_audio_length", False) else -1
    y = istft(merged, n_fft, hop, win, length, True, norm)
    return y.reshape(B, stems, ch, -1)


def bsroformer_forward(cfg: dict, w: dict, audio) -> np.ndarray:
    """BSRoformer::forward (model_bs_roformer.cu:420-609) composed from the
    functions above.  cfg: the checkpoint config; w: name -> fp32 array (the
    reference's weight names); audio [B, ch, S] -> [B, stems, ch, S']."""
    ch = np.shape(audio)[1]
    dims = [2 * f * ch for f in cfg["freqs_per_bands"]]
    return _roformer_forward(cfg, w, audio, dims, None, cfg.get("depth", 12),
                             cfg.get("mask_estimator_depth", 1), False, w["final_norm.gamma"])


def melbandroformer_forward(cfg: dict, w: dict, audio) -> np.ndarray:
    """MelBandRoformer::forward (model_mel_band_roformer.cu:745-1040): bands
    from w["__precomputed__.freq_indices"] / ["__precomputed__.num_freqs_per_band"]
    when present (model_mel_band_roformer.cu:322-375), else mel_bands; a norm
    closing every transformer (layers.{d}.{t}.norm.gamma), no final norm, and
    mask_estimator_depth + 1 linears per band MLP."""
    ch = np.shape(audio)[1]
    if "__precomputed__.freq_indices" in w:
        fidx = np.asarray(w["__precomputed__.freq_indices"], np.int64)
        counts = np.asarray(w["__precomputed__.num_freqs_per_band"], np.int64)
    else:
        fidx, counts = mel_bands(cfg.get("sample_rate", 44100), cfg.get("stft_n_fft", 2048),
                                 cfg.get("num_bands", 60), ch)
    dims = [int(2 * c * ch) for c in counts]
    return _roformer_forward(cfg, w, audio, dims, fidx, cfg.get("depth", 6),
                             cfg.get("mask_estimator_depth", 2) + 1, True, None)


def process_chunked(audio, chunk_size: int, step: int, batch: int, forward) -> np.ndarray:
    """The chunked driver (inference_app.cpp:100-324, Generic mode) in numpy:
    audio [ch, S]; forward maps [b, ch, chunk] -> [b, ..., n]."""
    audio = _f32(audio)
    C, S = audio.shape
    fade_size = chunk_size // 10
    border = chunk_size - step
    mix = audio
    padded = S > 2 * border and border > 0
    if padded:
        mix = np.pad(audio, ((0, 0), (border, border)), mode="reflect")
    total = mix.shape[1]
    starts = list(range(0, total, step))
    fade = np.ones(chunk_size, np.float32)
    if fade_size == 1:
        fade[0] = fade[-1] = 0.0
    elif fade_size > 1:
        a = (np.arange(fade_size) / (fade_size - 1)).astype(np.float32)
        fade[:fade_size] = a
        fade[-fade_size:] = 1.0 - a
    out, wsum = None, np.zeros(total, np.float32)
    for g in range(0, len(starts), max(1, min(batch, len(starts)))):
        group = starts[g:g + batch]
        chunks = []
        for st in group:
            c = mix[:, st:st + chunk_size]
            actual = c.shape[1]
            if actual < chunk_size:
                mode = "reflect" if actual > chunk_size // 2 else "constant"
                c = np.pad(c, ((0, 0), (0, chunk_size - actual)), mode=mode)
            chunks.append(c)
        y = forward(np.stack(chunks))
        n = y.shape[-1]
        y = y.reshape(len(group), -1, n)
        if out is None:
            out = np.zeros((y.shape[1], total), np.float32)
        for l, st in enumerate(group):
            actual = min(chunk_size, total - st)
            wnd = fade.copy()
            if fade_size > 0 and st == 0:
                wnd[:fade_size] = 1.0
            if fade_size > 0 and st + chunk_size >= total:
                wnd[-fade_size:] = 1.0
            m = min(actual, n)
            out[:, st:st + m] += y[l, :, :m] * wnd[:m]
            wsum[st:st + m] += wnd[:m]
    out = np.where(wsum > 1e-8, out / np.where(wsum > 1e-8, wsum, 1.0), out)
    return out[:, border:border + S] if padded else out
