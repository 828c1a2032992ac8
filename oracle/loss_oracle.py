"""CPU restatement of the trainer's reconstruction loss, in float64 numpy.

Test infrastructure only: tests/, __graft_entry__.smoke() and bench.py's CPU
baseline use it as the checker; the product never imports it.

Follows gaussian_splatting/utils/loss.py:12-33 of kmurungi/custom-3dgs-cuda:
    loss = (1 - lambda) * mean|gt - rendered| + lambda * (1 - SSIM)
with SSIM on the images clamped to [0, 1] (loss.py:8-10, ``_to_nchw``), as
torchmetrics' ``structural_similarity_index_measure`` computes it with the
reference's arguments (loss.py:30, data_range=1.0) and defaults: a Gaussian
window of 11 taps and sigma 1.5 (the 1D kernel exp(-(d/sigma)^2/2) over
d = -5..5, normalised to sum 1, used separably), K1 = 0.01, K2 = 0.03,
C1 = (K1 L)^2, C2 = (K2 L)^2, L = 1, the moments mu = w * x,
sigma_x^2 = max(w * x^2 - mu_x^2, 0) (torchmetrics clamps both variances at 0
since its releases after 1.0; 1.0 itself did not, which differs only where a
variance rounds below 0), sigma_xy = w * xy - mu_x mu_y, and the index
((2 mu_x mu_y + C1)(2 sigma_xy + C2)) / ((mu_x^2 + mu_y^2 + C1)(sigma_x^2 +
sigma_y^2 + C2)) averaged over channels and window centres (Wang et al. 2004).
torchmetrics pads by reflection and crops the index map by the window radius
afterwards; after that crop only windows lying wholly inside the image
remain, so this restatement evaluates exactly those ("valid" windows).  The
crop is torchmetrics' border handling as its source reads; no torchmetrics is
importable here to check it against, so that one choice is "parity unpinned"
(the test test_oracle_loss.py::test_padded_then_cropped_equals_valid shows the
padding cannot matter once the crop is made).
"""

from __future__ import annotations

import numpy as np

WINDOW = 11
SIGMA = 1.5
K1, K2 = 0.01, 0.03
C1, C2 = K1 * K1, K2 * K2
LAMBDA_DSSIM = 0.2  # loss.py:4


def gaussian_window(size: int = WINDOW, sigma: float = SIGMA) -> np.ndarray:
    d = np.arange(size, dtype=np.float64) - (size - 1) / 2.0
    g = np.exp(-0.5 * (d / sigma) ** 2)
    return g / g.sum()


def _blur_valid(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """Separable correlation of [H, W, C] with the 1D window along both axes,
    windows inside the image only: [H - k + 1, W - k + 1, C]."""
    k = w.size
    H, W = a.shape[:2]
    h = sum(w[j] * a[:, j:W - k + 1 + j] for j in range(k))
    return sum(w[i] * h[i:H - k + 1 + i] for i in range(k))


def _moments(x: np.ndarray, y: np.ndarray):
    w = gaussian_window()
    mx, my = _blur_valid(x, w), _blur_valid(y, w)
    exx, eyy, exy = _blur_valid(x * x, w), _blur_valid(y * y, w), _blur_valid(x * y, w)
    return mx, my, exx, eyy, exy


def _clamp0(v: np.ndarray) -> np.ndarray:
    """torch.clamp(v, min=0): NaN stays NaN."""
    return np.where(v < 0.0, 0.0, v)


def ssim_map(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """The SSIM index of each valid window and channel of two [H, W, 3] images
    (already in the data range): [H - 10, W - 10, 3]."""
    x, y = np.asarray(a, np.float64), np.asarray(b, np.float64)
    mx, my, exx, eyy, exy = _moments(x, y)
    sxx, syy, sxy = _clamp0(exx - mx * mx), _clamp0(eyy - my * my), exy - mx * my
    return ((2 * mx * my + C1) * (2 * sxy + C2)) / ((mx * mx + my * my + C1) * (sxx + syy + C2))


def ssim(a: np.ndarray, b: np.ndarray) -> float:
    return float(ssim_map(a, b).mean())


def clamp01(a: np.ndarray) -> np.ndarray:
    return np.clip(np.asarray(a, np.float64), 0.0, 1.0)


def l1_dssim(rendered, gt, lambda_dssim: float = LAMBDA_DSSIM) -> tuple[float, float, float]:
    """(loss, SSIM, L1 mean) of loss.py:12-33."""
    r, g = np.asarray(rendered, np.float64), np.asarray(gt, np.float64)
    l1 = float(np.mean(np.abs(g - r)))
    s = ssim(clamp01(r), clamp01(g))
    return (1.0 - lambda_dssim) * l1 + lambda_dssim * (1.0 - s), s, l1


def index_derivatives(mx, my, exx, eyy, exy):
    """The SSIM index S of windows with moments (mu_x, mu_y, E[x^2], E[y^2],
    E[xy]) and its partial derivatives (dS/dmu_x, dS/dE[x^2], dS/dE[xy]).  The
    clamp of sigma_x^2 at 0 passes its gradient where sigma_x^2 >= 0 (torch's
    clamp backward)."""
    vxx = exx - mx * mx
    sxx, syy, sxy = _clamp0(vxx), _clamp0(eyy - my * my), exy - mx * my
    a1, a2 = 2 * mx * my + C1, 2 * sxy + C2
    b1, b2 = mx * mx + my * my + C1, sxx + syy + C2
    s = a1 * a2 / (b1 * b2)
    dA1, dA2, dB1, dB2 = a2 / (b1 * b2), a1 / (b1 * b2), -s / b1, -s / b2
    dBx = np.where(vxx >= 0.0, dB2, 0.0)
    g1 = 2 * my * (dA1 - dA2) + 2 * mx * (dB1 - dBx)  # dS/dmu_x (through sigma_x^2, sigma_xy)
    g2 = dBx                                          # dS/dE[x^2]
    g3 = 2 * dA2                                      # dS/dE[xy]
    return s, g1, g2, g3


def _blur_adjoint(m: np.ndarray, w: np.ndarray, H: int, W: int) -> np.ndarray:
    """Adjoint of _blur_valid: each window centre's value spread back over its
    11 x 11 support, [H - 10, W - 10, C] -> [H, W, C]."""
    k = w.size
    h = np.zeros((m.shape[0], W) + m.shape[2:])
    for j in range(k):
        h[:, j:j + m.shape[1]] += w[j] * m
    out = np.zeros((H, W) + m.shape[2:])
    for i in range(k):
        out[i:i + m.shape[0]] += w[i] * h
    return out


def l1_dssim_grad(rendered, gt, lambda_dssim: float = LAMBDA_DSSIM, grad_loss: float = 1.0,
                  with_abs: bool = False):
    """d loss / d rendered [H, W, 3] in float64, by the chain rule through the
    SSIM index's moments: dS/dx_p = sum over windows q covering p of
    w(q - p) (dS_q/dmu_x + 2 x_p dS_q/dE[x^2] + y_p dS_q/dE[xy]); zero through
    the clamp where rendered is outside [0, 1] (torch's clamp backward passes
    it at 0 and 1); the L1 term -sgn(gt - rendered) / n.  With ``with_abs``
    also the sum of |terms| that formed each element."""
    r, g = np.asarray(rendered, np.float64), np.asarray(gt, np.float64)
    H, W = r.shape[:2]
    x, y = clamp01(r), clamp01(g)
    s, g1, g2, g3 = index_derivatives(*_moments(x, y))
    w = gaussian_window()
    n_win = s.size
    mask = (r >= 0.0) & (r <= 1.0)
    b_1, b_2, b_3 = (_blur_adjoint(m, w, H, W) for m in (g1, g2, g3))
    ds = (b_1 + 2 * x * b_2 + y * b_3) * mask
    n_px = r.size
    sg = -np.sign(g - r)
    grad = grad_loss * ((1 - lambda_dssim) / n_px * sg - lambda_dssim / n_win * ds)
    if not with_abs:
        return grad
    ab = (np.abs(_blur_adjoint(np.abs(g1), w, H, W)) + 2 * x * _blur_adjoint(np.abs(g2), w, H, W)
          + y * _blur_adjoint(np.abs(g3), w, H, W)) * mask
    absum = abs(grad_loss) * ((1 - lambda_dssim) / n_px * np.abs(sg) + lambda_dssim / n_win * ab)
    return grad, absum
