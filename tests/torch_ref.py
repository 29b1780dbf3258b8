"""Independent float64 restatement of the Roformer layer with torch library
routines, used to pin the C oracle (test infrastructure).

It is deliberately written differently from the oracle: RMSNorm through
F.normalize, RoPE as a complex rotation (torch.polar), attention through
F.scaled_dot_product_attention, GELU through F.gelu, heads through
reshape/permute.  Each function names the reference behaviour it encodes
(CUDA-MSST-Infer src/ file:line).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def t64(a):
    return torch.as_tensor(np.asarray(a), dtype=torch.float64)


def linear(x, w, b=None, act="none"):
    """nn.Linear then activation: ops_linear.cu:150-193, ops_fused.cu:264-303."""
    y = F.linear(t64(x), t64(w), None if b is None else t64(b))
    if act == "gelu":
        y = F.gelu(y)  # exact erf form, ops_fused.cu:21-24
    elif act == "sigmoid":
        y = torch.sigmoid(y)
    elif act == "silu":
        y = F.silu(y)
    return y


def rms_norm(x, gamma, scale):
    """x / sqrt(sum x^2) * gamma * scale  (ops_norm.cu:85-111).  F.normalize
    clamps the norm at eps instead of adding eps inside the sqrt; the two
    agree to ~1e-12 relative on non-degenerate rows."""
    x = t64(x)
    return F.normalize(x, dim=-1, eps=1e-30) * t64(gamma) * scale


def rope_angles(n, dh):
    """Angles n * 10000^(-2i/dh) in float64 (model_bs_roformer.cu:205-230)."""
    i = torch.arange(dh // 2, dtype=torch.float64)
    inv = 10000.0 ** (-2.0 * i / dh)
    return torch.outer(torch.arange(n, dtype=torch.float64), inv)


def rope(x, angles):
    """Interleaved pairs (2i, 2i+1) as complex numbers times e^{i theta}
    (ops_misc.cu:39-69).  x: [..., N, D]; angles: [N, D/2]."""
    x = t64(x)
    z = torch.view_as_complex(x.reshape(*x.shape[:-1], -1, 2).contiguous())
    rot = torch.polar(torch.ones_like(angles), angles)
    return torch.view_as_real(z * rot).reshape(x.shape)


def attention(q, k, v, scale=None):
    """softmax(scale q k^T) v  (ops_attention.cu:522-599)."""
    return F.scaled_dot_product_attention(t64(q), t64(k), t64(v), scale=scale)


def transformer(x, w, heads, dim_head, angles):
    """One Roformer transformer (attention + feed-forward, optional final
    norm), model_bs_roformer.cu:236-331 / model_mel_band_roformer.cu:519-651.
    x: [B, N, dim]; w: dict of numpy weights."""
    x = t64(x)
    B, N, dim = x.shape
    s = math.sqrt(dim)
    h = rms_norm(x, w["attn_gamma"], s)
    qkv = linear(h, w["w_qkv"])
    qkv = qkv.reshape(B, N, 3, heads, dim_head).permute(2, 0, 3, 1, 4)
    q, k, v = qkv[0], qkv[1], qkv[2]
    q = rope(q, angles)
    k = rope(k, angles)
    o = attention(q, k, v, scale=1.0 / math.sqrt(dim_head))
    g = linear(h, w["w_gate"], w["b_gate"], "sigmoid")          # [B, N, H]
    o = o * g.permute(0, 2, 1).unsqueeze(-1)
    o = o.permute(0, 2, 1, 3).reshape(B, N, heads * dim_head)
    x = x + linear(o, w["w_out"])
    h = rms_norm(x, w["ff_gamma"], s)
    h = linear(h, w["w_ff1"], w["b_ff1"], "gelu")
    x = x + linear(h, w["w_ff2"], w["b_ff2"])
    if w.get("final_gamma") is not None:
        x = rms_norm(x, w["final_gamma"], s)
    return x


def stack(x, layers, heads, dim_head, final_gamma=None):
    """Axial stack on x [B, T, F, dim] (model_bs_roformer.cu:482-539)."""
    x = t64(x)
    B, T, Fb, dim = x.shape
    ta = rope_angles(T, dim_head)
    fa = rope_angles(Fb, dim_head)
    for d in range(len(layers) // 2):
        xt = x.permute(0, 2, 1, 3).reshape(B * Fb, T, dim)
        xt = transformer(xt, layers[2 * d], heads, dim_head, ta)
        x = xt.reshape(B, Fb, T, dim).permute(0, 2, 1, 3)
        xf = x.reshape(B * T, Fb, dim)
        xf = transformer(xf, layers[2 * d + 1], heads, dim_head, fa)
        x = xf.reshape(B, T, Fb, dim)
    if final_gamma is not None:
        x = rms_norm(x, final_gamma, math.sqrt(dim))
    return x


def random_layer(rng, dim, heads, dim_head, ff, final_norm=False, dtype=np.float32):
    """Seeded weights: matrices and biases ~ N(0, 0.02), RMSNorm gammas
    1 + N(0, 0.02) (ones-init perturbed, so every layer keeps its scale)."""
    hd = heads * dim_head

    def n(*shape):
        return (rng.standard_normal(shape) * 0.02).astype(dtype)

    def g(d):
        return (1.0 + rng.standard_normal(d) * 0.02).astype(np.float32)

    w = dict(
        attn_gamma=g(dim), w_qkv=n(3 * hd, dim), w_gate=n(heads, dim),
        b_gate=n(heads).astype(np.float32), w_out=n(dim, hd), ff_gamma=g(dim),
        w_ff1=n(ff, dim), b_ff1=n(ff).astype(np.float32), w_ff2=n(dim, ff),
        b_ff2=n(dim).astype(np.float32), final_gamma=g(dim) if final_norm else None)
    return w
