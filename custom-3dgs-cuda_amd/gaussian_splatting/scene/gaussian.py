"""Gaussian parameter container; layouts of gaussian_splatting/scene/gaussian.py:3-12."""

import torch as t


class gaussian:
    """N Gaussians: means, (w,x,y,z) quaternions, log-scales, opacity logits,
    SH DC ("albedo") and the 15 x 3 band-1..3 SH coefficients."""

    def __init__(self, N: int) -> None:
        self.N = N
        self.mu = t.zeros(N, 3, dtype=t.float32)
        self.q = t.zeros(N, 4, dtype=t.float32)
        self.s = t.zeros(N, 3, dtype=t.float32)
        self.alpha = t.zeros(N, 1, dtype=t.float32)
        self.A = t.zeros(N, 3, dtype=t.float32)
        self.k_j = t.zeros(N, 15, 3, dtype=t.float32)
