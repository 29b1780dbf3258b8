"""Python binding of the MI355X Roformer hot path (libmsst_hip.so, C ABI in
include/msst_hip.h).

This module is plumbing for tests and the benchmark: it loads the in-tree
shared library with ctypes and passes torch device tensors to it as raw
pointers on torch's current HIP stream.  There is no fallback: if the
library is not built, `lib()` raises.

The package directory name contains dashes, so it is loaded by path:

    spec = importlib.util.spec_from_file_location(
        "msst_amd", "<repo>/cuda-msst-infer_amd/__init__.py",
        submodule_search_locations=["<repo>/cuda-msst-infer_amd"])
"""
from __future__ import annotations

import ctypes
import os
import subprocess

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libmsst_hip.so")

F32, F16 = 0, 1
ACT = {"none": 0, "gelu": 1, "sigmoid": 2, "silu": 3}

_lib = None


class MsstError(RuntimeError):
    pass


def build(jobs: int = 8) -> None:
    """Compile the HIP kernels and the C ABI for gfx950 (hipcc)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", PKG_DIR], check=True)


_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f = ctypes.c_float


class SeqLayout(ctypes.Structure):
    _fields_ = [(n, _i64) for n in (
        "n_outer", "n_inner", "seq_len", "tok_outer", "tok_inner", "tok_pos")]


class LayerWeights(ctypes.Structure):
    _fields_ = [(n, _vp) for n in (
        "attn_gamma", "w_qkv", "w_gate", "b_gate", "w_out", "ff_gamma",
        "w_ff1", "b_ff1", "w_ff2", "b_ff2", "final_gamma")]


class StackDesc(ctypes.Structure):
    _fields_ = [(n, _i64) for n in (
        "batch", "frames", "bands", "dim", "heads", "dim_head", "ff_dim", "depth")] + [
        ("w_dtype", _int)]


class BandConfig(ctypes.Structure):
    _fields_ = [("num_bands", _int), ("band_dims", ctypes.POINTER(_int)), ("dim", _int),
                ("hidden", _int), ("mlp_linears", _int), ("audio_channels", _int),
                ("stft_bins", _int), ("freq_indices", ctypes.POINTER(_int))]


_BCP = ctypes.POINTER(BandConfig)
_P64 = ctypes.POINTER(_i64)
_PP = ctypes.POINTER(_vp)

_SIGS = {
    "msst_abi_version": ([], _int),
    "msst_status_string": ([_int], ctypes.c_char_p),
    "msst_last_error": ([], ctypes.c_char_p),
    "msst_linear": ([_vp, _int, _vp, _int, _vp, _vp, _vp, _int, _i64, _i64, _i64, _int, _vp], _int),
    "msst_linear_rope": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _i64, _i64,
                          _i64, _vp], _int),
    "msst_rms_norm": ([_vp, _int, _vp, _f, _vp, _int, _i64, _i64, _vp], _int),
    "msst_rms_norm_gate": ([_vp, _int, _vp, _f, _vp, _int, _vp, _int, _vp, _vp, _i64, _i64,
                            _int, _vp], _int),
    "msst_rope_table": ([_int, _int, _vp, _vp], _int),
    "msst_rope_table_device": ([_int, _int, _vp, _vp, _vp], _int),
    "msst_rope_qk": ([_vp, _vp, _int, _vp, _vp, _i64, _i64, _i64, _i64, _vp], _int),
    "msst_attention": ([_vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _i64, _f, _vp], _int),
    "msst_gated_rope_attention": ([_vp, _int, _i64, _vp, _vp, _vp, _vp, _i64,
                                   ctypes.POINTER(SeqLayout), _int, _int, _f, _vp], _int),
    "msst_split_qkv_heads": ([_vp, _vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _vp], _int),
    "msst_gate_merge_heads": ([_vp, _vp, _vp, _int, _i64, _i64, _i64, _i64, _vp], _int),
    "msst_cast": ([_vp, _int, _vp, _int, _i64, _vp], _int),
    "msst_add": ([_vp, _vp, _vp, _int, _i64, _vp], _int),
    "msst_swap_axes12": ([_vp, _vp, _int, _i64, _i64, _i64, _i64, _vp], _int),
    "msst_roformer_stack_workspace": ([ctypes.POINTER(StackDesc)], _i64),
    "msst_roformer_stack": ([_vp, ctypes.POINTER(StackDesc), ctypes.POINTER(LayerWeights), _vp,
                             _vp, _i64, _vp], _int),
    "msst_tanh": ([_vp, _vp, _int, _i64, _vp], _int),
    "msst_glu": ([_vp, _vp, _int, _i64, _i64, _vp], _int),
    "msst_band_plan_bytes": ([_BCP], _i64),
    "msst_band_plan_init": ([_BCP, _PP, _PP, _PP, _PP, _PP, _vp, _i64, _vp], _int),
    "msst_band_split_workspace": ([_BCP, _i64], _i64),
    "msst_band_split": ([_BCP, _vp, _vp, _i64, _vp, _vp, _i64, _vp], _int),
    "msst_mask_estimator_workspace": ([_BCP, _i64], _i64),
    "msst_mask_estimator": ([_BCP, _vp, _vp, _int, _i64, _vp, _vp, _i64, _vp], _int),
    "msst_band_gather": ([_BCP, _vp, _vp, _i64, _i64, _vp, _vp], _int),
    "msst_mask_merge_workspace": ([_BCP, _i64, _i64, _i64], _i64),
    "msst_mask_merge": ([_BCP, _vp, _vp, _i64, _vp, _i64, _i64, _int, _vp, _vp, _i64, _vp], _int),
    "msst_chunk_extract": ([_vp, _i64, _i64, _i64, _i64, _i64, _int, _vp, _vp], _int),
    "msst_overlap_add": ([_vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp], _int),
    "msst_normalize_by_weights": ([_vp, _vp, _i64, _i64, _vp], _int),
    "msst_stft_frames": ([_i64, _int, _int, _int], _i64),
    "msst_stft": ([_vp, _i64, _i64, _int, _int, _vp, _int, _int, _vp, _vp], _int),
    "msst_istft_length": ([_i64, _int, _int, _i64, _int], _i64),
    "msst_istft_workspace": ([_i64, _i64, _int], _i64),
    "msst_istft": ([_vp, _i64, _i64, _int, _int, _vp, _i64, _int, _int, _vp, _vp, _i64, _vp], _int),
    "msst_hann_window": ([_vp, _int, _vp], _int),
    "msst_roformer_transformer": ([_vp, ctypes.POINTER(StackDesc), ctypes.POINTER(LayerWeights),
                                   _int, _vp, _i64, _vp], _int),
    "msst_roformer_stack_noalloc": ([_vp, ctypes.POINTER(StackDesc), ctypes.POINTER(LayerWeights),
                                     _vp, _vp], _int),
    "msst_complex_mul": ([_vp, _vp, _vp, _i64, _vp], _int),
    "msst_roformer_stack_layer": ([_vp, ctypes.POINTER(StackDesc), ctypes.POINTER(LayerWeights),
                                   _int, _vp, _i64, _vp], _int),
    "msst_strided_copy": ([_vp, _P64, _vp, _P64, _P64, _int, _int, _vp], _int),
    "msst_binary": ([_vp, _P64, _vp, _P64, _vp, _P64, _int, _int, _int, _vp], _int),
}

# Bytes of the library's own device scratch behind msst_roformer_stack_noalloc.
STACK_SCRATCH_BYTES = 64 << 20

EXPORTED = tuple(_SIGS)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MsstError(f"{LIB_PATH} is not built; run build() (hipcc, gfx950)")
        # RTLD_NOW: an unresolved symbol fails here, not at first call.
        l = ctypes.CDLL(LIB_PATH, mode=os.RTLD_NOW)
        for name, (args, res) in _SIGS.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = res
        _lib = l
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        l = lib()
        raise MsstError(f"{what}: {l.msst_status_string(rc).decode()} "
                        f"({rc}): {l.msst_last_error().decode()}")


# ---------------------------------------------------------------------------
# torch helpers (torch is imported lazily: the C ABI itself needs no torch).
# ---------------------------------------------------------------------------
def _dt(t) -> int:
    import torch
    if t.dtype == torch.float32:
        return F32
    if t.dtype == torch.float16:
        return F16
    raise MsstError(f"unsupported dtype {t.dtype}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def linear(x, w, bias=None, act="none", residual=None, out=None, out_dtype=None):
    """act(x . w^T + bias) (+ residual); returns `out` [.., N]."""
    import torch
    K = x.shape[-1]
    N = w.shape[0]
    M = x.numel() // K
    if out is None:
        od = out_dtype or (residual.dtype if residual is not None else torch.float32)
        out = torch.empty(*x.shape[:-1], N, dtype=od, device=x.device)
    check(lib().msst_linear(_ptr(x), _dt(x), _ptr(w), _dt(w), _ptr(bias), _ptr(residual),
                            _ptr(out), _dt(out), M, K, N, ACT[act], _stream()), "msst_linear")
    return out


def linear_rope(x, w, cos, sin, rope_cols, dim_head, pos_div, pos_mod, bias=None, out=None):
    """fp16 x . w^T (+ bias) with RoPE on columns [0, rope_cols); row r is at
    position (r // pos_div) % pos_mod of the [pos_mod, dim_head/2] tables."""
    import torch
    K = x.shape[-1]
    N = w.shape[0]
    M = x.numel() // K
    if out is None:
        out = torch.empty(*x.shape[:-1], N, dtype=torch.float16, device=x.device)
    check(lib().msst_linear_rope(_ptr(x), _ptr(w), _ptr(bias), _ptr(out), M, K, N, _ptr(cos),
                                 _ptr(sin), rope_cols, dim_head, pos_div, pos_mod, _stream()),
          "msst_linear_rope")
    return out


def rms_norm(x, gamma, scale, out=None, out_dtype=None):
    import torch
    D = x.shape[-1]
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
    check(lib().msst_rms_norm(_ptr(x), _dt(x), _ptr(gamma), float(scale), _ptr(out), _dt(out),
                              x.numel() // D, D, _stream()), "msst_rms_norm")
    return out


def rms_norm_gate(x, gamma, scale, w_gate, b_gate, out_dtype=None, out=None, gates=None):
    import torch
    D = x.shape[-1]
    rows = x.numel() // D
    G = w_gate.shape[0]
    if out is None:
        out = torch.empty(x.shape, dtype=out_dtype or x.dtype, device=x.device)
    if gates is None:
        gates = torch.empty(*x.shape[:-1], G, dtype=torch.float32, device=x.device)
    check(lib().msst_rms_norm_gate(_ptr(x), _dt(x), _ptr(gamma), float(scale), _ptr(out),
                                   _dt(out), _ptr(w_gate), _dt(w_gate), _ptr(b_gate),
                                   _ptr(gates), rows, D, G, _stream()), "msst_rms_norm_gate")
    return out, gates


def rope_table(n: int, dim_head: int):
    import numpy as np
    c = np.empty((n, dim_head // 2), np.float32)
    s = np.empty((n, dim_head // 2), np.float32)
    check(lib().msst_rope_table(n, dim_head, c.ctypes.data_as(_vp), s.ctypes.data_as(_vp)),
          "msst_rope_table")
    return c, s


def rope_table_device(n: int, dim_head: int, device="cuda"):
    import torch
    c = torch.empty(n, dim_head // 2, dtype=torch.float32, device=device)
    s = torch.empty_like(c)
    check(lib().msst_rope_table_device(n, dim_head, _ptr(c), _ptr(s), _stream()),
          "msst_rope_table_device")
    return c, s


def rope_qk_(q, k, cos_t, sin_t):
    B, H, N, D = q.shape
    check(lib().msst_rope_qk(_ptr(q), _ptr(k), _dt(q), _ptr(cos_t), _ptr(sin_t), B, H, N, D,
                             _stream()), "msst_rope_qk")


def attention(q, k, v, scale=0.0):
    import torch
    B, H, N, D = q.shape
    Nk = k.shape[2]
    out = torch.empty_like(q)
    check(lib().msst_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(out), _dt(q), B, H, N, Nk, D,
                               float(scale), _stream()), "msst_attention")
    return out


def seq_layout(n_outer, n_inner, seq_len, tok_outer, tok_inner, tok_pos) -> SeqLayout:
    return SeqLayout(n_outer, n_inner, seq_len, tok_outer, tok_inner, tok_pos)


def gated_rope_attention(qkv, layout: SeqLayout, heads, cos_t=None, sin_t=None, gates=None,
                         scale=0.0, out=None):
    import torch
    D = qkv.shape[-1] // (3 * heads)
    tokens = qkv.numel() // qkv.shape[-1]
    if out is None:
        out = torch.empty(tokens, heads * D, dtype=qkv.dtype, device=qkv.device)
    check(lib().msst_gated_rope_attention(_ptr(qkv), _dt(qkv), qkv.shape[-1], _ptr(cos_t),
                                          _ptr(sin_t), _ptr(gates), _ptr(out), out.shape[-1],
                                          ctypes.byref(layout), heads, D, float(scale),
                                          _stream()), "msst_gated_rope_attention")
    return out


def split_qkv_heads(qkv, heads):
    import torch
    B, N, C = qkv.shape
    D = C // (3 * heads)
    q = torch.empty(B, heads, N, D, dtype=qkv.dtype, device=qkv.device)
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    check(lib().msst_split_qkv_heads(_ptr(qkv), _ptr(q), _ptr(k), _ptr(v), _dt(qkv), B, N, heads,
                                     D, _stream()), "msst_split_qkv_heads")
    return q, k, v


def gate_merge_heads(attn, gates):
    import torch
    B, H, N, D = attn.shape
    out = torch.empty(B, N, H * D, dtype=attn.dtype, device=attn.device)
    check(lib().msst_gate_merge_heads(_ptr(attn), _ptr(gates), _ptr(out), _dt(attn), B, H, N, D,
                                      _stream()), "msst_gate_merge_heads")
    return out


def cast(x, dtype):
    import torch
    out = torch.empty(x.shape, dtype=dtype, device=x.device)
    check(lib().msst_cast(_ptr(x), _dt(x), _ptr(out), _dt(out), x.numel(), _stream()),
          "msst_cast")
    return out


def add(a, b, out=None):
    import torch
    if out is None:
        out = torch.empty_like(a)
    check(lib().msst_add(_ptr(a), _ptr(b), _ptr(out), _dt(a), a.numel(), _stream()), "msst_add")
    return out


def swap_axes12(x):
    """[A,P,Q,R] -> [A,Q,P,R] (new tensor)."""
    import torch
    A, P, Q, R = x.shape
    out = torch.empty(A, Q, P, R, dtype=x.dtype, device=x.device)
    check(lib().msst_swap_axes12(_ptr(x), _ptr(out), _dt(x), A, P, Q, R, _stream()),
          "msst_swap_axes12")
    return out


class RoformerStack:
    """Device-resident weights of an axial Roformer stack and its workspace.

    layers: list of dicts (time0, freq0, time1, freq1, ...) holding torch
    device tensors under the msst_layer_weights field names; matrices in the
    stack dtype, gammas/biases fp32.  Mirrors the transformer part of
    BSRoformer / MelBandRoformer (model_bs_roformer.cu:482-539).
    """

    def __init__(self, layers, final_gamma, batch, frames, bands, dim, heads, dim_head,
                 ff_dim, w_dtype):
        import torch
        self.layers = layers
        self.final_gamma = final_gamma
        self.desc = StackDesc(batch, frames, bands, dim, heads, dim_head, ff_dim,
                              len(layers) // 2, w_dtype)
        ws = lib().msst_roformer_stack_workspace(ctypes.byref(self.desc))
        if ws < 0:
            check(-1, "msst_roformer_stack_workspace")
        self.workspace = torch.empty(int(ws), dtype=torch.uint8, device="cuda")
        arr = (LayerWeights * len(layers))()
        for i, lw in enumerate(layers):
            for name, _ in LayerWeights._fields_:
                t = lw.get(name)
                setattr(arr[i], name, None if t is None else t.data_ptr())
        self._arr = arr

    def __call__(self, x):
        """In place on x [batch, frames, bands, dim] fp32 (device)."""
        check(lib().msst_roformer_stack(_ptr(x), ctypes.byref(self.desc), self._arr,
                                        _ptr(self.final_gamma), _ptr(self.workspace),
                                        self.workspace.numel(), _stream()),
              "msst_roformer_stack")
        return x

    def call_noalloc(self, x):
        """Like __call__, through msst_roformer_stack_noalloc: the library's
        own device scratch instead of self.workspace."""
        check(lib().msst_roformer_stack_noalloc(_ptr(x), ctypes.byref(self.desc), self._arr,
                                                _ptr(self.final_gamma), _stream()),
              "msst_roformer_stack_noalloc")
        return x

    def layer(self, x, layer: int, axis: int):
        """One transformer in place on x [batch, frames, bands, dim] fp32 (the
        stack's layout); axis 0 = time, 1 = frequency."""
        check(lib().msst_roformer_stack_layer(
            _ptr(x), ctypes.byref(self.desc), ctypes.byref(self._arr[layer]), axis,
            _ptr(self.workspace), self.workspace.numel(), _stream()),
            "msst_roformer_stack_layer")
        return x

    def transformer(self, x, layer: int, axis: int):
        """One transformer in place on x [batch, bands, frames, dim] fp32
        (time-major); axis 0 = time, 1 = frequency."""
        check(lib().msst_roformer_transformer(
            _ptr(x), ctypes.byref(self.desc), ctypes.byref(self._arr[layer]), axis,
            _ptr(self.workspace), self.workspace.numel(), _stream()),
            "msst_roformer_transformer")
        return x


def hann_window(size: int, device="cuda"):
    import torch
    out = torch.empty(size, device=device)
    check(lib().msst_hann_window(_ptr(out), size, _stream()), "msst_hann_window")
    return out


def stft(signal, n_fft, hop, window, center=True, normalized=False):
    """signal f32 [B, L] -> [B, n_fft/2 + 1, T, 2] (torch.stft semantics)."""
    import torch
    B, L = signal.shape
    T = lib().msst_stft_frames(L, n_fft, hop, int(center))
    if T < 1:
        raise MsstError("msst_stft_frames: n_fft must be a power of two in [16, 4096], hop >= 1, "
                        "and the signal long enough for one frame (centre: L > n_fft / 2)")
    out = torch.empty(B, n_fft // 2 + 1, T, 2, device=signal.device)
    check(lib().msst_stft(_ptr(signal), B, L, n_fft, hop, _ptr(window), int(center),
                          int(normalized), _ptr(out), _stream()), "msst_stft")
    return out


def istft(spec, n_fft, hop, window, length=-1, center=True, normalized=False):
    """spec f32 [B, n_fft/2 + 1, T, 2] -> [B, out_len] (torch.istft semantics)."""
    import torch
    B, F, T, _ = spec.shape
    n = lib().msst_istft_length(T, n_fft, hop, length, int(center))
    if n < 1:
        raise MsstError("msst_istft_length: bad n_fft / hop / frames / length")
    out = torch.empty(B, n, device=spec.device)
    wsb = lib().msst_istft_workspace(B, T, n_fft)
    ws = torch.empty(max(int(wsb), 16), dtype=torch.uint8, device=spec.device)
    check(lib().msst_istft(_ptr(spec), B, T, n_fft, hop, _ptr(window), length, int(center),
                           int(normalized), _ptr(out), _ptr(ws), wsb, _stream()), "msst_istft")
    return out


def tanh(x, out=None):
    import torch
    if out is None:
        out = torch.empty_like(x)
    check(lib().msst_tanh(_ptr(x), _ptr(out), _dt(x), x.numel(), _stream()), "msst_tanh")
    return out


def glu(x):
    """Last-axis GLU: x[..., :n] * sigmoid(x[..., n:])."""
    import torch
    half = x.shape[-1] // 2
    out = torch.empty(*x.shape[:-1], half, dtype=x.dtype, device=x.device)
    check(lib().msst_glu(_ptr(x), _ptr(out), _dt(x), x.numel() // (2 * half), half, _stream()),
          "msst_glu")
    return out


class BandPlan:
    """Device plan of the band split and/or one stem's mask estimator
    (msst_band_plan_init).  dims: features per band; split = (gammas, ws,
    biases) per band; mask = (ws, biases) per band, each a list of the L
    linears.  Keeps references to every tensor it points at."""

    def __init__(self, dims, dim, split=None, mask=None, hidden=0, channels=0, stft_bins=0,
                 freq_indices=None):
        import torch
        self.dims = [int(d) for d in dims]
        self._dims_c = (_int * len(self.dims))(*self.dims)
        L = len(mask[0][0]) if mask is not None else 1
        if mask is not None and L > 1:
            hidden = mask[0][0][0].shape[0]
        self._fidx_c = None
        if freq_indices is not None:
            self._fidx_c = (_int * len(freq_indices))(*[int(v) for v in freq_indices])
        self.channels, self.stft_bins = int(channels), int(stft_bins)
        self.cfg = BandConfig(len(self.dims), self._dims_c, int(dim), int(hidden), int(L),
                              self.channels, self.stft_bins, self._fidx_c)
        nbytes = lib().msst_band_plan_bytes(ctypes.byref(self.cfg))
        if nbytes < 0:
            check(-2, "msst_band_plan_bytes")
        self.plan = torch.empty(int(nbytes), dtype=torch.uint8, device="cuda")
        self._keep = []

        def arr(ts):
            if ts is None:
                return None
            self._keep.extend(ts)
            return (_vp * len(ts))(*[t.data_ptr() for t in ts])

        sg = sw = sb = mw = mb = None
        if split is not None:
            sg, sw, sb = (arr(list(x)) for x in split)
        if mask is not None:
            mw = arr([w for band in mask[0] for w in band])
            mb = arr([b for band in mask[1] for b in band])
        check(lib().msst_band_plan_init(ctypes.byref(self.cfg), sg, sw, sb, mw, mb,
                                        _ptr(self.plan), nbytes, _stream()),
              "msst_band_plan_init")

    def band_split(self, x, out=None):
        """x f32 [rows, sum(dims)] -> f32 [rows, nb, dim]."""
        import torch
        rows = x.shape[0]
        if out is None:
            out = torch.empty(rows, len(self.dims), self.cfg.dim, device=x.device)
        wsb = lib().msst_band_split_workspace(ctypes.byref(self.cfg), rows)
        ws = torch.empty(max(int(wsb), 1), dtype=torch.uint8, device=x.device)
        check(lib().msst_band_split(ctypes.byref(self.cfg), _ptr(self.plan), _ptr(x), rows,
                                    _ptr(out), _ptr(ws), wsb, _stream()), "msst_band_split")
        return out

    def mask_estimator(self, x, out=None):
        """x f32/f16 [rows, nb, dim] -> f32 [rows, sum(dims)]."""
        import torch
        rows = x.shape[0]
        if out is None:
            out = torch.empty(rows, sum(self.dims), device=x.device)
        wsb = lib().msst_mask_estimator_workspace(ctypes.byref(self.cfg), rows)
        ws = torch.empty(max(int(wsb), 1), dtype=torch.uint8, device=x.device)
        check(lib().msst_mask_estimator(ctypes.byref(self.cfg), _ptr(self.plan), _ptr(x), _dt(x),
                                        rows, _ptr(out), _ptr(ws), wsb, _stream()),
              "msst_mask_estimator")
        return out

    def band_gather(self, stft, batch):
        """stft f32 [batch * ch, F, T, 2] -> band features f32 [batch, T, sum(dims)]."""
        import torch
        T = stft.shape[2]
        out = torch.empty(batch, T, sum(self.dims), device=stft.device)
        check(lib().msst_band_gather(ctypes.byref(self.cfg), _ptr(self.plan), _ptr(stft), batch,
                                     T, _ptr(out), _stream()), "msst_band_gather")
        return out

    def mask_merge(self, masks, stft, batch, zero_dc=True):
        """masks f32 [stems, batch, T, sum(dims)], stft f32 [batch * ch, F, T, 2]
        -> masked STFT f32 [batch * stems * ch, F, T, 2]."""
        import torch
        stems, T = masks.shape[0], stft.shape[2]
        out = torch.empty(batch * stems * self.channels, self.stft_bins, T, 2, device=stft.device)
        wsb = lib().msst_mask_merge_workspace(ctypes.byref(self.cfg), batch, stems, T)
        ws = torch.empty(max(int(wsb), 16), dtype=torch.uint8, device=stft.device)
        check(lib().msst_mask_merge(ctypes.byref(self.cfg), _ptr(self.plan), _ptr(masks), stems,
                                    _ptr(stft), batch, T, int(bool(zero_dc)), _ptr(out), _ptr(ws),
                                    wsb, _stream()), "msst_mask_merge")
        return out
