"""Fits the polynomial coefficients of the noise kernel's inverse normal CDF.

The device evaluates z = sqrt(2) * erfinv(x) as x * P(L) with L =
log2(1 - x^2), the variable substitution of M. Giles, "Approximating the
erfinv function" (GPU Computing Gems, Jade Edition, 2011): erfinv(x) / x is
smooth in log(1 - x^2), so one polynomial covers the centre and a second one,
in sqrt(-L), the tails.  The coefficients here are this project's own fit
(near-minimax relative error by Lawson's iteratively reweighted least squares
on Chebyshev nodes, against scipy's float64 erfinv); they are pasted into
odp_noise.hip.  Run: python opaque_amd/csrc/fit_icdf.py

The kernel's input x is (k - 2^23) * 2^-23 for a 24-bit uniform k, and it
multiplies the float (k - 2^23) by P directly, so P = sqrt(2) erfinv(x) /
x * 2^-23.  The self-check below compares with scipy's erfinv directly.
"""

from __future__ import annotations

import numpy as np
from numpy.polynomial import chebyshev as cheb
from scipy.special import erfinv

L_SPLIT = -8.0  # centre: L in [L_SPLIT, 0]; tail: sqrt(-L) in [sqrt(-L_SPLIT), sqrt(L_MAX)]
L_MAX = 22.0  # 1 - x^2 >= 2^-21 for the clamped 24-bit uniforms; a margin beyond
DEG_CENTRE = 8
DEG_TAIL = 7
SCALE = 2.0**-23  # ratio() already carries sqrt(2)


def ratio(L: np.ndarray) -> np.ndarray:
    """sqrt(2) * erfinv(x) / x where 1 - x^2 = 2^L (float64)."""
    x = np.sqrt(-np.expm1(L * np.log(2.0)))
    out = np.full_like(L, np.sqrt(2.0) * np.sqrt(np.pi) / 2.0)
    big = x > 1e-7
    out[big] = np.sqrt(2.0) * erfinv(x[big]) / x[big]
    return out


def fit(lo: float, hi: float, deg: int, fun) -> np.ndarray:
    """Monomial coefficients (lowest first) of a near-minimax relative fit on [lo, hi]."""
    t = np.cos(np.pi * (np.arange(40000) + 0.5) / 40000)
    v = lo + (hi - lo) * (t + 1.0) / 2.0
    y = fun(v)
    w = 1.0 / np.abs(y)
    for _ in range(60):
        c = cheb.chebfit(t, y, deg, w=w)
        err = np.abs((cheb.chebval(t, c) - y) / y)
        w = w * (1.0 + 20.0 * err / err.max())
    p = np.polynomial.Chebyshev(c, domain=[lo, hi]).convert(kind=np.polynomial.Polynomial)
    return p.coef


def horner_f32(coef: np.ndarray, v: np.ndarray) -> np.ndarray:
    """Horner in float32 with fused multiply-adds (as the device evaluates it)."""
    v32 = v.astype(np.float32).astype(np.float64)
    acc = np.full(v.shape, np.float32(coef[-1]), dtype=np.float32)
    for c in coef[-2::-1]:
        acc = (acc.astype(np.float64) * v32 + np.float64(np.float32(c))).astype(np.float32)
    return acc


def main() -> None:
    centre = fit(L_SPLIT, 0.0, DEG_CENTRE, ratio) * SCALE
    s_lo, s_hi = np.sqrt(-L_SPLIT), np.sqrt(L_MAX)
    mid = float(np.float32((s_lo + s_hi) / 2.0))
    tail = fit(s_lo - mid, s_hi - mid, DEG_TAIL, lambda t: ratio(-((t + mid) ** 2))) * SCALE

    L = np.linspace(L_SPLIT, 0.0, 400001)
    e_c = np.abs(horner_f32(centre, L) / (ratio(L) * SCALE) - 1.0).max()
    s = np.linspace(s_lo, s_hi, 400001).astype(np.float32)
    ts = (s - np.float32(mid)).astype(np.float32)
    e_t = np.abs(horner_f32(tail, ts.astype(np.float64)) / (ratio(-(s.astype(np.float64) ** 2)) * SCALE) - 1.0).max()
    # End-to-end check on x directly: z = xf * P(log2(1 - x^2)) against
    # sqrt(2) * erfinv(x) for x on the 24-bit grid.
    k = np.arange(2, 2**24 - 1, 97, dtype=np.int64)
    xf = (k - 2**23).astype(np.float64)
    x = xf * 2.0**-23
    Lx = np.log2(1.0 - x * x)
    pz = np.where(Lx >= L_SPLIT, horner_f32(centre, Lx),
                  horner_f32(tail, np.sqrt(-Lx).astype(np.float32) - np.float32(mid)))
    want = np.sqrt(2.0) * erfinv(x)
    nz = want != 0
    e_x = np.abs(xf[nz] * pz[nz] / want[nz] - 1.0).max()
    assert e_x < 5e-7, e_x
    print(f"// fit_icdf.py: centre max rel err {e_c:.2e} (L in [{L_SPLIT}, 0]), "
          f"tail {e_t:.2e} (sqrt(-L) in [{s_lo:.4f}, {s_hi:.4f}]); against erfinv on the grid {e_x:.2e}")
    print(f"constexpr float ICDF_L_SPLIT = {L_SPLIT:.1f}f;")
    print(f"constexpr float ICDF_TAIL_MID = {mid:.9e}f;")
    for name, coef in (("ICDF_CENTRE", centre), ("ICDF_TAIL", tail)):
        body = ", ".join(f"{np.float32(c):.9e}f" for c in coef)
        print(f"constexpr float {name}[{len(coef)}] = {{{body}}};")


if __name__ == "__main__":
    main()
