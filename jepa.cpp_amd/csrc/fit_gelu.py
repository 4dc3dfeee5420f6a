"""Coefficients of the GELU used by the GEMM epilogues (gemm.hip: gelu_erf).

GELU(x) = 0.5 x (1 + erf(x / sqrt 2)) = x Phi(x), Phi the standard normal CDF. With t = |x| and the
tail h(t) = Phi(-t) = 0.5 erfc(t / sqrt 2):
    Phi(x) = 1 - h(t) for x >= 0,   h(t) for x < 0,
    h(t)   = 2^Q(min(t, T)),        Q of degree 8 ~ log2(h) on [0, T], T = 5.5,
one polynomial and one hardware exp2 for every x (no second branch to evaluate and select). Q is fitted
with weight h(t), so the absolute error of h, which is the absolute error of Phi on both sides, is what
is minimised. At T, h = 1.9e-8 < 2^-25, so 1 - h rounds to exactly 1.0f and GELU(x) = x for x >= T.
Least squares on Chebyshev nodes, reweighted toward equal ripple. Prints the float32 coefficients and
the largest absolute error of Phi from the float32 evaluation (fma per Horner step; exp2 correctly
rounded, and off by two units either way) against scipy's double erfc.  Run: python fit_gelu.py
"""
import numpy as np
from scipy.special import erfc

T, DEG = 5.5, 8
f32 = np.float32


def fma32(a, b, c):
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(f32)


def cheb(lo, hi, n):
    return (np.cos(np.linspace(0, np.pi, n)) * 0.5 + 0.5) * (hi - lo) + lo


def fit():
    # Q(0) = -1 exactly (h(0) = 1/2, so Phi(0) = 1/2 without error): Q(t) = -1 + t R(t)
    t = cheb(0, T, 8000)
    h = 0.5 * erfc(t / np.sqrt(2))
    V = np.vander(t, DEG + 1, increasing=True)[:, 1:]
    f = np.log2(h) + 1
    c, *_ = np.linalg.lstsq(V * h[:, None], f * h, rcond=None)
    for _ in range(30):
        e = (V @ c - f) * h
        w = h * (1 + 50 * np.abs(e) / np.abs(e).max())
        c, *_ = np.linalg.lstsq(V * w[:, None], f * w, rcond=None)
    return np.concatenate([[-1.0], c]).astype(f32)


def phi32(x, c, ulps=0):
    x = x.astype(f32)
    t = np.minimum(np.abs(x), f32(T))
    q = np.full_like(t, c[-1])
    for a in c[-2::-1]:
        q = fma32(q, t, np.full_like(t, a))
    h = np.exp2(q.astype(np.float64)).astype(f32)
    for _ in range(abs(ulps)):
        h = np.nextafter(h, f32(np.inf) if ulps > 0 else f32(-np.inf)).astype(f32)
    return np.where(x >= 0, (f32(1) - h).astype(f32), h)


if __name__ == "__main__":
    c = fit()
    print("Q (t^0 .. t^8):", ", ".join("%.9ef" % a for a in c))
    xs = np.concatenate([np.linspace(-8, 8, 2_000_001), np.geomspace(1e-8, 8, 200000),
                         -np.geomspace(1e-8, 8, 200000)]).astype(f32)
    exact = np.where(xs >= 0, 1 - 0.5 * erfc(xs.astype(np.float64) / np.sqrt(2)), 0.5 * erfc(-xs.astype(np.float64) / np.sqrt(2)))
    for u in (0, 2, -2):
        err = np.abs(phi32(xs, c, u).astype(np.float64) - exact)
        print("exp2 off by %+d units: max |Phi32 - Phi| = %.3e (%.2f units of 2^-24) at x = %.5f"
              % (u, err.max(), err.max() / 2.0 ** -24, xs[err.argmax()]))
