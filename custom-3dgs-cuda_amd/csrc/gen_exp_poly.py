"""Derivation of the exp polynomial used by exp_gs (gsr_common.h) and the oracle.

exp(x) = 2^k * e^r with k = rint(x * log2 e) and r = x - k*ln2 in [-ln2/2, ln2/2]
(Cody & Waite reduction; ln2 split as fdlibm's 0x3f317200 + 0x35bfbe8e, so k*ln2_hi
is exact).  e^r is approximated by 1 + c1 r + ... + c6 r^6.  The coefficients come
from a relative-error weighted least-squares fit on Chebyshev nodes, re-weighted
towards the minimax solution, then rounded to fp32.  Run to print them; the
faithful-rounding claim (max 0.955 ulp over [-87.34, 88.72]) is checked by
tests/test_oracle_exp.py on the compiled function.
"""

import numpy as np


def fit(deg: int = 6, npts: int = 4000, iters: int = 60) -> np.ndarray:
    half = np.log(2.0) / 2
    t = np.cos(np.pi * (np.arange(npts) + 0.5) / npts) * half
    A = np.stack([t ** k for k in range(1, deg + 1)], axis=1)
    b = np.exp(t) - 1.0
    w = 1.0 / np.exp(t)
    c, *_ = np.linalg.lstsq(A * w[:, None], b * w, rcond=None)
    for _ in range(iters):
        err = np.abs((A @ c - b) * w)
        w2 = w * (err / err.max() + 1e-3) ** 0.5
        c, *_ = np.linalg.lstsq(A * w2[:, None], b * w2, rcond=None)
        w = w2 / w2.max() * (1.0 / np.exp(t)).max()
    return c


if __name__ == "__main__":
    c = fit()
    half = np.log(2.0) / 2
    t = np.linspace(-half, half, 200001)
    c32 = c.astype(np.float32).astype(np.float64)
    approx = 1 + sum(c32[k - 1] * t ** k for k in range(1, len(c32) + 1))
    print("max relative error of the fp32 coefficients on the reduced range:",
          np.max(np.abs(approx / np.exp(t) - 1)))
    for k, v in enumerate(c.astype(np.float32), start=1):
        print(f"c{k} = {float(v)!r}  ({np.float32(v).view(np.uint32):#010x})")
