"""Regenerates the GELU coefficients of gelu_erf (msst_common.hpp).

c(a) = Phi(-a) is approximated as 2^P(min(a, A)) with P of degree 6 and
A = 5.6.  P is the minimax fit of log2 Phi(-a) in the first-order absolute
error of c, |2^P - c| ~ c ln2 |P - log2 c|, on 3000 points of [0, A]: a
linear program in the seven coefficients and the error bound.  The script
then evaluates the kernel's expression in float32 (FMA with one rounding,
exp2 off by +-1 ulp) against float64 v Phi(v) and prints the worst error
relative to |v|.  Run: python gelu_fit.py (numpy + scipy).
"""
import numpy as np
from scipy.optimize import linprog
from scipy.special import ndtr

DEGREE, A, POINTS = 6, 5.6, 3000


def fit():
    a = np.linspace(0.0, A, POINTS)
    c = ndtr(-a)
    y, w = np.log2(c), c * np.log(2.0)
    V = np.vander(a, DEGREE + 1, increasing=True)
    cost = np.zeros(DEGREE + 2)
    cost[-1] = 1.0
    ones = np.ones((POINTS, 1))
    A_ub = np.block([[w[:, None] * V, -ones], [-w[:, None] * V, -ones]])
    b_ub = np.concatenate([w * y, -w * y])
    r = linprog(cost, A_ub=A_ub, b_ub=b_ub, bounds=[(None, None)] * (DEGREE + 2), method="highs")
    assert r.success, r.message
    return np.float32(r.x[:-1]), r.x[-1]


def kernel_expr(coef, v, exp_ulps):
    f32 = lambda t: np.asarray(t, dtype=np.float64).astype(np.float32)
    v = f32(v)
    a = np.abs(v)
    x = np.minimum(a, np.float32(A))
    p = np.full_like(x, coef[-1])
    for k in range(DEGREE - 1, -1, -1):
        p = f32(p.astype(np.float64) * x + np.float64(coef[k]))
    c = f32(np.exp2(p.astype(np.float64)) * (1.0 + exp_ulps * 2.0**-23))
    return f32(a.astype(np.float64) * f32(0.5 - c.astype(np.float64)) + f32(0.5 * v.astype(np.float64)))


if __name__ == "__main__":
    coef, bound = fit()
    print(f"degree {DEGREE} on [0, {A}]: |error of c| <= {bound:.2e}")
    for k in range(DEGREE, -1, -1):
        print(f"  c{k} = {float(coef[k])!r}f")
    v = np.concatenate([np.linspace(-40, 40, 4_000_001), np.geomspace(1e-38, 1e38, 20000),
                        -np.geomspace(1e-38, 1e38, 20000)]).astype(np.float32)
    v = v[v != 0]
    exact = v.astype(np.float64) * ndtr(v.astype(np.float64))
    worst = 0.0
    for ulps in (-1.0, 0.0, 1.0):
        err = np.abs(kernel_expr(coef, v, ulps).astype(np.float64) - exact) / np.abs(v.astype(np.float64))
        worst = max(worst, float(np.max(err)))
    print(f"worst |gelu - v Phi(v)| / |v| = {worst:.2e}")
