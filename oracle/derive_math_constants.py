"""Derives the polynomial coefficients of the oracle's (and kernel's) expf / logf.

TEST INFRASTRUCTURE / provenance only: nothing imports this module.  Run it to
reproduce the fp32 bit patterns hard-coded in oracle/mdq_oracle.c and
stream-mm2026_amd/csrc/mdq_math.h.

Method: minimax fits by Lawson's algorithm (iteratively reweighted least
squares on Chebyshev nodes) in float64 against mpmath at 40 digits, then the
coefficients are rounded to fp32.
  log: (log1p(r) - r) / r^2 on r in [c - 1, 2c - 1), c = 0x3f2aaaab (~2/3), degree 8
  exp: (e^r - 1 - r) / r^2 on |r| <= ln2/2, degree 5
The resulting functions were then measured exhaustively against float64
(tests/test_oracle_math.py): log 0.974 ulp, exp 0.988 ulp max error.
"""
import struct

import numpy as np
from mpmath import mp

mp.dps = 40


def lawson(f, a, b, deg, n=4000, iters=400):
    x = np.cos(np.linspace(0, np.pi, n)) * (b - a) / 2 + (a + b) / 2
    y = np.array([f(t) for t in x])
    w = np.ones(n) / n
    V = np.vander(x, deg + 1, increasing=True)
    for _ in range(iters):
        sw = np.sqrt(w)
        c, *_ = np.linalg.lstsq(V * sw[:, None], y * sw, rcond=None)
        e = np.abs(V @ c - y)
        w = w * e
        w /= w.sum()
    return c, float(np.max(np.abs(V @ c - y)))


def log_aux(r):
    r_ = mp.mpf(r)
    if abs(r) < 1e-6:
        return float(-mp.mpf(1) / 2 + r_ / 3 - r_ ** 2 / 4 + r_ ** 3 / 5)
    return float((mp.log1p(r_) - r_) / r_ ** 2)


def exp_aux(r):
    r_ = mp.mpf(r)
    if abs(r) < 1e-6:
        return float(mp.mpf(1) / 2 + r_ / 6 + r_ ** 2 / 24 + r_ ** 3 / 120)
    return float((mp.exp(r_) - 1 - r_) / r_ ** 2)


def f32hex(v):
    return "0x%08x" % struct.unpack("<I", struct.pack("<f", np.float32(v)))[0]


def main():
    c = float(np.float32(struct.unpack("<f", struct.pack("<I", 0x3F2AAAAB))[0]))
    co, err = lawson(log_aux, c - 1.0, 2 * c - 1.0, 8)
    print("log  P(r), degree 8, max fit error %.3g:" % err, [f32hex(v) for v in co])
    ln2 = float(mp.log(2))
    co, err = lawson(exp_aux, -ln2 / 2 - 1e-4, ln2 / 2 + 1e-4, 5)
    print("exp  E(r), degree 5, max fit error %.3g:" % err, [f32hex(v) for v in co])


if __name__ == "__main__":
    main()
