"""Derives the erfc coefficients of the fp16 / bf16 GELU kernel (activation.hip).

erfc(z) = t * exp(-z^2 + P(t)),  t = 1 / (1 + z/2),  z >= 0,

with P a degree-9 polynomial: the Chebyshev interpolant, on 4000 nodes of
t in (0, 1], of P*(t) = log(erfc(z) / t) + z^2 = log(erfcx(z) / t)
(z = 2 (1 - t) / t; scipy's erfcx avoids the underflow of erfc).  The form is
the classic one of Numerical Recipes' erfcc; these coefficients are fitted
here.  Prints them (float32, highest degree first, for Horner's rule) and the
largest |P - P*| on a fine grid, which is the relative error of erfc before
fp32 rounding: about 1.0e-7.
"""
import numpy as np
import scipy.special as sp
from numpy.polynomial import chebyshev as C
from numpy.polynomial import polynomial as P


def target(t):
    z = 2 * (1 - t) / t
    return np.log(sp.erfcx(z) / t)


def fit(deg: int = 9, nodes: int = 4000):
    k = np.arange(nodes)
    t = 0.5 * (1 + np.cos((2 * k + 1) * np.pi / (2 * nodes)))
    t = t[t > 1e-6]
    cheb = C.chebfit(2 * t - 1, target(t), deg)
    in_s = C.cheb2poly(cheb)               # polynomial in s = 2t - 1
    in_t = np.zeros(1)
    for i, c in enumerate(in_s):
        in_t = P.polyadd(in_t, c * P.polypow([-1, 2], i))
    return in_t.astype(np.float32)


if __name__ == "__main__":
    coef = fit()
    grid = np.linspace(1e-6, 1, 200001)
    err = np.abs(P.polyval(grid, coef.astype(np.float64)) - target(grid)).max()
    for c in coef[::-1]:
        print(f"{float(c):.9e}f,")
    print(f"max |P - P*| = {err:.3e}")
