"""The GELU coefficients in msst_common.hpp (gelu_erf) against their fit.

gelu_fit.py (beside the kernels) fits log2 Phi(-a) on [0, 5.6] by a linear
program; the header holds the float32-rounded coefficients.  This checks that
the header's constants are that fit's, and that the kernel's expression with
them, evaluated in float32 with v_exp_f32 off by one ulp either way, stays
within the 2.4e-7 |v| stated in the header, over all finite v.
"""
import importlib.util
import pathlib
import re

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
CSRC = ROOT / "cuda-msst-infer_amd" / "csrc"


def _fit_module():
    spec = importlib.util.spec_from_file_location("gelu_fit", CSRC / "gelu_fit.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _header_coefficients():
    """c0 .. c6 as written in gelu_erf: fmaf(x, c6, c5), then fmaf(x, p, c_k), k = 4 .. 0."""
    src = (CSRC / "msst_common.hpp").read_text()
    body = src[src.index("float gelu_erf(float v)"):]
    body = body[:body.index("\n}\n")]
    first = re.search(r"fmaf\(x,\s*([-+0-9.eE]+)f,\s*([-+0-9.eE]+)f\)", body)
    rest = re.findall(r"fmaf\(x,\s*p,\s*([-+0-9.eE]+)f\)", body)
    high_to_low = [float(first.group(1)), float(first.group(2))] + [float(c) for c in rest]
    return np.float32(high_to_low[::-1])


def test_header_coefficients_are_the_fit():
    pytest.importorskip("scipy")
    fit = _fit_module()
    coef, bound = fit.fit()
    assert bound < 1e-7
    hdr = _header_coefficients()
    assert hdr.shape == coef.shape == (7,)
    np.testing.assert_allclose(hdr, coef, rtol=1e-5, atol=1e-9)


def test_gelu_expression_error_bound():
    pytest.importorskip("scipy")
    from scipy.special import ndtr
    fit = _fit_module()
    coef = _header_coefficients()
    v = np.concatenate([np.linspace(-40, 40, 2_000_001), np.geomspace(1e-38, 1e38, 20000),
                        -np.geomspace(1e-38, 1e38, 20000)]).astype(np.float32)
    v = v[v != 0]
    exact = v.astype(np.float64) * ndtr(v.astype(np.float64))
    for ulps in (-1.0, 0.0, 1.0):
        g = fit.kernel_expr(coef, v, ulps).astype(np.float64)
        assert np.max(np.abs(g - exact) / np.abs(v.astype(np.float64))) <= 2.4e-7
    with np.errstate(all="ignore"):
        special = fit.kernel_expr(coef, np.float32([np.inf, -np.inf, np.nan, 0.0]), 0.0)
    assert special[0] == np.inf and np.isnan(special[1]) and np.isnan(special[2])
    assert special[3] == 0.0
