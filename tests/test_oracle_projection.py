"""Pins of the oracle's projection forward/backward (projection.cu:33-105,
projection_backward.cu:33-138) against closed forms and finite differences."""

import numpy as np

# The reference's 0.3f anti-aliasing term, as the fp32 literal it is.
AA = float(np.float32(0.3))


def _rot_np(q):
    """Rotation of a unit quaternion (w,x,y,z), written independently of the oracle
    (the standard matrix; the reference restates it at utils/adc.py:105-114)."""
    w, x, y, z = q / np.linalg.norm(q)
    return np.array([
        [1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y)],
        [2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x)],
        [2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)],
    ])


def _ewa_np(mu, q, s, Rc, t, fx, fy, cx, cy):
    """Textbook EWA splatting: mean, J Rc R S^2 R^T Rc^T J^T + 0.3 I, depth."""
    out_m, out_c, out_d = [], [], []
    for m, qq, ss in zip(mu, q, s):
        pc = Rc @ m + t
        if pc[2] <= 0.2:
            out_m.append([0, 0]); out_c.append([0, 0, 0]); out_d.append(0)
            continue
        x, y, z = pc
        R = _rot_np(qq)
        Sw = R @ np.diag(np.exp(2 * ss)) @ R.T
        Sc = Rc @ Sw @ Rc.T
        J = np.array([[fx / z, 0, -fx * x / z ** 2], [0, fy / z, -fy * y / z ** 2]])
        C = J @ Sc @ J.T
        out_m.append([fx * x / z + cx, fy * y / z + cy])
        out_c.append([C[0, 0] + AA, C[0, 1], C[1, 1] + AA])
        out_d.append(z)
    return np.array(out_m), np.array(out_c), np.array(out_d)


def _random_pose(rng):
    Rc = _rot_np(rng.normal(size=4))
    t = rng.normal(size=3) * 0.2 + np.array([0, 0, 0.5])
    return Rc, t


def _inputs(rng, n=64):
    mu = np.c_[rng.uniform(-1, 1, (n, 2)), rng.uniform(1.0, 6.0, n)]
    q = rng.normal(size=(n, 4))
    s = rng.normal(-3.0, 0.7, (n, 3))
    return mu, q, s


def test_identity_isotropic_closed_form(orc):
    # identity q, isotropic s, identity camera: Sigma_cam = sigma^2 I, so
    # a = sigma^2 (J00^2 + J02^2) + 0.3, b = sigma^2 J02 J12, c = sigma^2 (J11^2 + J12^2) + 0.3
    rng = np.random.default_rng(0)
    n = 100
    # fp32-representable inputs, so the fp32 path sees the same values
    mu = np.c_[rng.uniform(-1, 1, (n, 2)), rng.uniform(1.0, 6.0, n)].astype(np.float32).astype(np.float64)
    q = np.tile([1.0, 0, 0, 0], (n, 1))
    s = np.repeat(rng.normal(-3, 0.5, (n, 1)), 3, axis=1).astype(np.float32).astype(np.float64)
    fx, fy, cx, cy = 500.0, 450.0, 320.0, 240.0
    x, y, z = mu.T
    sig2 = np.exp(2 * s[:, 0])
    J00, J02, J11, J12 = fx / z, -fx * x / z ** 2, fy / z, -fy * y / z ** 2
    want_c = np.c_[sig2 * (J00 ** 2 + J02 ** 2) + AA, sig2 * J02 * J12, sig2 * (J11 ** 2 + J12 ** 2) + AA]
    want_m = np.c_[fx * x / z + cx, fy * y / z + cy]
    for dt, tol in ((np.float64, 1e-12), (np.float32, 2e-6)):
        m2, c2, d = orc.project(mu, q, s, np.eye(3), np.zeros(3), fx, fy, cx, cy, dtype=dt)
        np.testing.assert_allclose(m2, want_m, rtol=tol)
        np.testing.assert_allclose(c2, want_c, rtol=tol, atol=tol * 10)
        np.testing.assert_allclose(d, z, rtol=tol)


def test_general_pose_matches_textbook_ewa(orc):
    rng = np.random.default_rng(1)
    mu, q, s = _inputs(rng)
    Rc, t = _random_pose(rng)
    want = _ewa_np(mu, q, s, Rc, t, 400.0, 380.0, 200.0, 150.0)
    got = orc.project(mu, q, s, Rc, t, 400.0, 380.0, 200.0, 150.0, dtype=np.float64)
    for g, w in zip(got, want):
        np.testing.assert_allclose(g, w, rtol=1e-10, atol=1e-10)


def test_culled_gaussians_are_zero(orc):
    mu = np.array([[0.0, 0.0, 0.2], [0.0, 0.0, -1.0], [0.1, 0.1, 0.2000001]])
    q = np.tile([1.0, 0, 0, 0], (3, 1))
    s = np.full((3, 3), -2.0)
    m2, c2, d = orc.project(mu, q, s, np.eye(3), np.zeros(3), 100.0, 100.0, 50.0, 50.0)
    assert np.all(m2[:2] == 0) and np.all(c2[:2] == 0) and np.all(d[:2] == 0)
    assert d[2] > 0.2 and c2[2, 0] > 0.3


def test_zero_quaternion_is_identity(orc):
    # glm::normalize returns the identity quaternion for a zero-length quaternion
    mu = np.array([[0.1, -0.2, 3.0]] * 2)
    q = np.array([[0.0, 0, 0, 0], [1.0, 0, 0, 0]])
    s = np.array([[-2.0, -2.5, -3.0]] * 2)
    _, c2, _ = orc.project(mu, q, s, np.eye(3), np.zeros(3), 200.0, 200.0, 0, 0)
    np.testing.assert_array_equal(c2[0], c2[1])


def _fd_project(orc, mu, q, s, Rc, t, cam, wm, wc, which, eps=1e-6):
    base = {"mu": mu, "q": q, "s": s}
    x = base[which]
    g = np.zeros_like(x)
    for idx in np.ndindex(*x.shape):
        vals = []
        for sgn in (1, -1):
            xp = x.copy()
            xp[idx] += sgn * eps
            args = dict(base)
            args[which] = xp
            m2, c2, _ = orc.project(args["mu"], args["q"], args["s"], Rc, t, *cam, dtype=np.float64)
            vals.append(np.sum(wm * m2) + np.sum(wc * c2))
        g[idx] = (vals[0] - vals[1]) / (2 * eps)
    return g


def test_backward_matches_finite_differences_fp64(orc):
    rng = np.random.default_rng(2)
    mu, q, s = _inputs(rng, n=12)
    Rc, t = _random_pose(rng)
    cam = (420.0, 400.0, 210.0, 160.0)
    wm, wc = rng.normal(size=(12, 2)), rng.normal(size=(12, 3))
    dmu, dq, ds = orc.project_bwd(wm, wc, mu, q, s, Rc, t, *cam, dtype=np.float64)
    for name, got in (("mu", dmu), ("q", dq), ("s", ds)):
        want = _fd_project(orc, mu, q, s, Rc, t, cam, wm, wc, name)
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max(),
                                   err_msg=name)


def test_reference_literal_quaternion_formula_fails_finite_differences(orc):
    """projection_backward.cu:116-127 read literally (ref_quat=True) is not the
    derivative of the forward rotation; it fails the same finite-difference check."""
    rng = np.random.default_rng(3)
    mu, q, s = _inputs(rng, n=8)
    cam = (420.0, 400.0, 210.0, 160.0)
    wm, wc = rng.normal(size=(8, 2)), rng.normal(size=(8, 3))
    _, dq_ref, _ = orc.project_bwd(wm, wc, mu, q, s, np.eye(3), np.zeros(3), *cam,
                                   dtype=np.float64, ref_quat=True)
    want = _fd_project(orc, mu, q, s, np.eye(3), np.zeros(3), cam, wm, wc, "q")
    rel = np.abs(dq_ref - want).max() / np.abs(want).max()
    assert rel > 0.1


def test_reference_gradcheck_scene_fp32(orc):
    """tests/test_cuda_backward.py:53-113 (2 Gaussians, fx=fy=200, cx=cy=100) with the
    reference's gradcheck tolerances (eps 1e-3, atol 1e-3, rtol 1e-2), full Jacobian of
    the fp32 backward against central differences of the forward."""
    mu = np.array([[0.30, -0.20, 3.5], [-0.25, 0.15, 5.0]], np.float32)
    quat = np.array([1.0, 0.15, -0.05, 0.02], np.float32)
    quat = quat / np.linalg.norm(quat)
    q = np.tile(quat, (2, 1)).astype(np.float32)
    s = np.array([[-2.2, -2.0, -1.8], [-2.5, -2.1, -2.3]], np.float32)
    cam = (200.0, 200.0, 100.0, 100.0)
    R, t = np.eye(3, dtype=np.float32), np.zeros(3, np.float32)
    m2, c2, _ = orc.project(mu, q, s, R, t, *cam)
    assert np.all(np.isfinite(m2)) and np.abs(m2).sum() > 1.0 and np.abs(c2).sum() > 0.1
    inputs = {"mu": mu, "q": q, "s": s}
    n_out = 2 * 2 + 2 * 3
    for name, x in inputs.items():
        ana = np.zeros((n_out, x.size))
        num = np.zeros((n_out, x.size))
        for o in range(n_out):
            wm = np.zeros((2, 2), np.float32)
            wc = np.zeros((2, 3), np.float32)
            (wm if o < 4 else wc).reshape(-1)[o if o < 4 else o - 4] = 1.0
            dmu, dq, ds = orc.project_bwd(wm, wc, mu, q, s, R, t, *cam)
            ana[o] = {"mu": dmu, "q": dq, "s": ds}[name].reshape(-1)
        for j in range(x.size):
            outs = []
            for sgn in (1, -1):
                xp = {k: v.copy() for k, v in inputs.items()}
                xp = {k: v.astype(np.float64) for k, v in xp.items()}
                xp[name].reshape(-1)[j] += sgn * 1e-3
                # central differences of the float64 forward at the fp32 inputs: an
                # fp32 forward differenced at eps 1e-3 carries ~ulp(c)/eps of noise
                a2, b2, _ = orc.project(xp["mu"], xp["q"], xp["s"], R, t, *cam, dtype=np.float64)
                outs.append(np.concatenate([a2.reshape(-1), b2.reshape(-1)]).astype(np.float64))
            num[:, j] = (outs[0] - outs[1]) / 2e-3
        bad = np.abs(ana - num) > 1e-3 + 1e-2 * np.abs(num)
        assert not bad.any(), (name, np.argwhere(bad)[:5], ana[bad][:5], num[bad][:5])
