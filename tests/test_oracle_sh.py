"""Pins of the oracle's SH colour forward/backward (SH.cu:12-91, delight_backward.cu:7-173)."""

import numpy as np

C0 = 0.28209479177387814


def _fib_sphere(n):
    i = np.arange(n) + 0.5
    phi = np.arccos(1 - 2 * i / n)
    th = np.pi * (1 + 5 ** 0.5) * i
    return np.c_[np.cos(th) * np.sin(phi), np.sin(th) * np.sin(phi), np.cos(phi)]


def test_dc_only_closed_form_bitwise(orc):
    rng = np.random.default_rng(0)
    n = 1000
    A = rng.uniform(-3, 3, (n, 3)).astype(np.float32)
    mu = rng.normal(size=(n, 3)).astype(np.float32) + np.float32(5)
    got = orc.sh(np.zeros(3), mu, A, np.zeros((n, 15, 3)))
    want = np.clip(np.float32(0.5) + np.float32(C0) * A, 0, 1)
    np.testing.assert_array_equal(got, want)


def test_basis_is_orthonormal_real_sh(orc):
    """The 15 band-1..3 functions plus the DC term C0 form an orthonormal set on the
    sphere: a wrong constant or a flipped cross term breaks the Gram matrix."""
    dirs = _fib_sphere(40000)
    n = dirs.shape[0]
    Y = np.zeros((n, 16))
    Y[:, 0] = C0
    for k in range(15):
        kj = np.zeros((n, 15, 3))
        kj[:, k, 0] = 0.1
        col = orc.sh(np.zeros(3), 3.0 * dirs, np.zeros((n, 3)), kj, dtype=np.float64)
        Y[:, k + 1] = (col[:, 0] - 0.5) / 0.1
    gram = 4 * np.pi * (Y.T @ Y) / n
    np.testing.assert_allclose(gram, np.eye(16), atol=2e-3)


def test_backward_matches_finite_differences_fp64(orc):
    rng = np.random.default_rng(1)
    n = 6
    mu = rng.normal(size=(n, 3)) + np.array([0, 0, 3.0])
    cam = np.array([0.1, -0.2, 0.05])
    A = rng.uniform(-0.3, 0.3, (n, 3))
    kj = rng.normal(0, 0.05, (n, 15, 3))
    w = rng.normal(size=(n, 3))
    col = orc.sh(cam, mu, A, kj, dtype=np.float64)
    assert np.all((col > 0.02) & (col < 0.98))  # inside the clamp
    dA, dkj, dmu = orc.sh_bwd(w, mu, A, kj, cam, dtype=np.float64)
    base = {"mu": mu, "A": A, "kj": kj}
    for name, got in (("mu", dmu), ("A", dA), ("kj", dkj)):
        x = base[name]
        num = np.zeros_like(x)
        for idx in np.ndindex(*x.shape):
            v = []
            for sgn in (1, -1):
                args = {k: a.copy() for k, a in base.items()}
                args[name][idx] += sgn * 1e-6
                v.append(np.sum(w * orc.sh(cam, args["mu"], args["A"], args["kj"], dtype=np.float64)))
            num[idx] = (v[0] - v[1]) / 2e-6
        np.testing.assert_allclose(got, num, rtol=1e-6, atol=1e-8, err_msg=name)


def test_clamp_mask_zeroes_gradient(orc):
    mu = np.array([[0.0, 0.0, 3.0]] * 3, np.float32)
    A = np.array([[10.0, -10.0, 0.0]] * 3, np.float32)  # r > 1, g < 0, b inside
    kj = np.zeros((3, 15, 3), np.float32)
    dA, dkj, dmu = orc.sh_bwd(np.ones((3, 3), np.float32), mu, A, kj, np.zeros(3, np.float32))
    assert np.all(dA[:, :2] == 0) and np.all(dA[:, 2] == np.float32(C0))
    assert np.all(dkj[:, :, :2] == 0)


def test_reference_gradcheck_scene_fp32(orc):
    """tests/test_cuda_backward.py:116-161: 2 Gaussians, camera at the origin, A = 0,
    k_j = linspace(-.005, .005); colours inside (0.05, 0.95); reference tolerances."""
    mu = np.array([[0.40, -0.30, 2.5], [-0.20, 0.50, 3.0]], np.float32)
    A = np.zeros((2, 3), np.float32)
    kj = np.linspace(-0.005, 0.005, 90, dtype=np.float32).reshape(2, 15, 3)
    cam = np.zeros(3, np.float32)
    col = orc.sh(cam, mu, A, kj)
    assert col.min() > 0.05 and col.max() < 0.95
    inputs = {"mu": mu, "A": A, "kj": kj}
    for name, x in inputs.items():
        ana = np.zeros((6, x.size))
        num = np.zeros((6, x.size))
        for o in range(6):
            w = np.zeros((2, 3), np.float32)
            w.reshape(-1)[o] = 1
            dA, dkj, dmu = orc.sh_bwd(w, mu, A, kj, cam)
            ana[o] = {"mu": dmu, "A": dA, "kj": dkj}[name].reshape(-1)
        for j in range(x.size):
            outs = []
            for sgn in (1, -1):
                xp = {k: v.astype(np.float64) for k, v in inputs.items()}
                xp[name].reshape(-1)[j] += sgn * 1e-3
                outs.append(orc.sh(cam, xp["mu"], xp["A"], xp["kj"], dtype=np.float64).reshape(-1))
            num[:, j] = (outs[0] - outs[1]) / 2e-3
        assert np.all(np.abs(ana - num) <= 1e-3 + 1e-2 * np.abs(num)), name
