"""Coefficients of the branch-free erf used by the GEMM's GELU epilogue (gemm.hip: erf_nonneg).

erf(z), z >= 0, in two pieces evaluated together and selected (no divergent branch):
  z <  ZB:  erf(z)  = z * P(z^2)          P of degree 5: relative error of erf(z)/z
  z >= ZB:  erfc(z) = 2^Q(min(z, 4))      Q of degree 6 ~ log2(erfc(z)), weighted by erfc(z) so that
                                          the absolute error of 1 - erfc(z) is what is minimised
(erfc(4) = 1.5e-8 rounds 1 - erfc to exactly 1.0f, as erff does for z > 3.92.)
Least squares on Chebyshev nodes, reweighted toward equal ripple. Prints the float32 coefficients
and the maximum absolute error of the float32 evaluation (fma per Horner step, hardware-like exp2)
against scipy's double erf on a dense sample.  Run: python fit_gelu_erf.py
"""
import math
import numpy as np
from scipy.special import erf, erfc

ZB, ZMAX, DS, DL = 0.875, 4.0, 5, 6
f32 = np.float32


def fma32(a, b, c):
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(f32)


def cheb(lo, hi, n):
    return (np.cos(np.linspace(0, np.pi, n)) * 0.5 + 0.5) * (hi - lo) + lo


def refit(V, f, w0):
    c, *_ = np.linalg.lstsq(V * w0[:, None], f * w0, rcond=None)
    for _ in range(30):
        e = (V @ c - f) * w0
        w = w0 * (1 + 50 * np.abs(e) / np.abs(e).max())
        c, *_ = np.linalg.lstsq(V * w[:, None], f * w, rcond=None)
    return c


def fit():
    s = cheb(0, ZB * ZB, 4000)
    z = np.sqrt(s)
    f = np.where(z > 0, erf(z) / np.where(z > 0, z, 1), 2 / math.sqrt(math.pi))
    cs = refit(np.vander(s, DS + 1, increasing=True), f, np.ones_like(s))
    z = cheb(ZB, ZMAX, 6000)
    cl = refit(np.vander(z, DL + 1, increasing=True), np.log2(erfc(z)), erfc(z))
    return cs.astype(f32), cl.astype(f32)


def erf32(z, cs, cl):
    z = z.astype(f32)
    s = (z * z).astype(f32)
    p = np.full_like(z, cs[-1])
    for a in cs[-2::-1]:
        p = fma32(p, s, np.full_like(z, a))
    small = (z * p).astype(f32)
    zc = np.minimum(z, f32(ZMAX))
    q = np.full_like(z, cl[-1])
    for a in cl[-2::-1]:
        q = fma32(q, zc, np.full_like(z, a))
    large = (f32(1) - np.exp2(q.astype(np.float64)).astype(f32)).astype(f32)
    return np.where(z < f32(ZB), small, large)


if __name__ == "__main__":
    cs, cl = fit()
    print("P (s^0 .. s^5, s = z^2):", ", ".join("%.9ef" % c for c in cs))
    print("Q (z^0 .. z^6):          ", ", ".join("%.9ef" % c for c in cl))
    rng = np.random.default_rng(0)
    zs = np.concatenate([np.linspace(0, 4.5, 2_000_001), rng.uniform(0, 4.5, 2_000_000),
                         np.geomspace(1e-8, 1, 100000)]).astype(f32)
    err = np.abs(erf32(zs, cs, cl).astype(np.float64) - erf(zs.astype(np.float64)))
    print("max |erf32 - erf| = %.3e (%.2f units of 2^-24) at z = %.5f" % (err.max(), err.max() / 2.0 ** -24, zs[err.argmax()]))
