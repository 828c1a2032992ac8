"""CPU pins of the checkpoint and PLY export pieces: the record oracle
(oracle/ply_oracle.py) against the reference's own torch operations on CPU
tensors (scripts/run.py:96-123: transpose + flatten, norm + clamp_min + divide,
clamp + log), the channel-major closed form, the file layout against the PLY
specification (ASCII header, binary little-endian float32 body) by a hand
parse, and the .pt checkpoint round trip (utils/saveweights.py:5-20,
scripts/run.py:55-63)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splatting.scene.gaussian import gaussian
from gaussian_splatting.utils.ply import attribute_names, ply_header, read_ply
from gaussian_splatting.utils.saveweights import load_gaussians, save_weights
from oracle import ply_oracle as po


def _cloud(n, seed=0, legacy=False, K=15):
    gen = torch.Generator().manual_seed(seed)
    g = gaussian(n)
    g.mu = torch.randn(n, 3, generator=gen)
    g.q = torch.randn(n, 4, generator=gen) * torch.exp(torch.randn(n, 1, generator=gen))
    g.q[::7] = 0.0
    g.s = torch.randn(n, 3, generator=gen) - 4.0
    g.alpha = (torch.rand(n, 1, generator=gen) * 0.98 + 0.01) if legacy else \
        torch.randn(n, 1, generator=gen) * 3.0
    g.A = torch.rand(n, 3, generator=gen)
    g.k_j = torch.randn(n, K, 3, generator=gen) * 0.1
    return g


def _reference_torch_records(g, max_sh_degree=3):
    """The reference's save_ply arithmetic (run.py:96-123) on CPU tensors."""
    n_rest = (max_sh_degree + 1) ** 2 - 1
    n = g.mu.shape[0]
    rest = g.k_j.float()
    if rest.shape[1] < n_rest:
        rest = torch.cat([rest, torch.zeros(n, n_rest - rest.shape[1], 3)], dim=1)
    elif rest.shape[1] > n_rest:
        rest = rest[:, :n_rest, :]
    f_rest = rest.transpose(1, 2).reshape(n, 3 * n_rest)
    alpha = g.alpha.float().reshape(n, 1)
    if bool(((alpha > 0.0) & (alpha < 1.0)).all()) and float(alpha.min()) > 1e-6:
        alpha = alpha.clamp(1e-6, 1.0 - 1e-6)
        opacity = torch.log(alpha / (1.0 - alpha))
    else:
        opacity = alpha
    quat = g.q.float().reshape(n, 4)
    quat = quat / quat.norm(dim=-1, keepdim=True).clamp_min(1e-8)
    return torch.cat([g.mu, torch.zeros(n, 3), g.A.reshape(n, 3), f_rest, opacity,
                      g.s.reshape(n, 3), quat], dim=1).numpy()


@pytest.mark.parametrize("legacy", [False, True])
@pytest.mark.parametrize("deg,K", [(3, 15), (1, 15), (4, 15), (3, 8)])
def test_record_oracle_matches_the_reference_ops(legacy, deg, K):
    g = _cloud(20_000, seed=deg * 10 + K, legacy=legacy, K=K)
    want = _reference_torch_records(g, deg)
    got = po.vertex_records(g.mu, g.q, g.s, g.alpha, g.A, g.k_j, deg)
    assert got.shape == want.shape == (20_000, 17 + 3 * ((deg + 1) ** 2 - 1))
    op = 9 + 3 * ((deg + 1) ** 2 - 1)
    cols = [i for i in range(got.shape[1]) if i != op]
    assert np.array_equal(got[:, cols].view(np.uint32), want[:, cols].view(np.uint32))
    # the opacity column: copies bit for bit; the legacy log within 1 ulp (torch's
    # CPU log is not correctly rounded; the oracle's is)
    d = np.abs(got[:, op].view(np.int32).astype(np.int64) - want[:, op].view(np.int32))
    assert d.max() <= (1 if legacy else 0)


def test_channel_major_closed_form():
    g = _cloud(100, seed=3)
    rec = po.vertex_records(g.mu, g.q, g.s, g.alpha, g.A, g.k_j)
    kj = g.k_j.numpy()
    names = attribute_names(15)
    for n in (0, 41, 99):
        for c in range(3):
            for k in range(15):
                assert rec[n, names.index(f"f_rest_{c * 15 + k}")] == kj[n, k, c]
    r = rec[:, names.index("rot_0"):]
    nz = np.abs(g.q.numpy()).sum(1) > 0
    assert np.allclose(np.linalg.norm(r[nz], axis=1), 1.0, atol=1e-6)
    assert np.all(r[~nz] == 0)


def test_ply_layout_by_the_specification(tmp_path):
    names = attribute_names(15)
    assert len(names) == 62 and names[:9] == ["x", "y", "z", "nx", "ny", "nz", "f_dc_0", "f_dc_1",
                                               "f_dc_2"]
    assert names[9] == "f_rest_0" and names[53] == "f_rest_44" and names[54] == "opacity"
    assert names[55:] == ["scale_0", "scale_1", "scale_2", "rot_0", "rot_1", "rot_2", "rot_3"]
    rec = np.random.default_rng(0).normal(size=(5, 62)).astype(np.float32)
    hdr = ply_header(5, names)
    text = hdr.decode("ascii")
    assert text.startswith("ply\nformat binary_little_endian 1.0\nelement vertex 5\n")
    assert text.endswith("property float rot_3\nend_header\n")
    assert text.count("\nproperty float ") == 62
    p = tmp_path / "x.ply"
    p.write_bytes(hdr + rec.astype("<f4").tobytes())
    raw = p.read_bytes()
    body = raw[len(hdr):]
    assert len(body) == 5 * 62 * 4
    # float32 little-endian, record-major: the third record's 'opacity'
    v = np.frombuffer(body, dtype="<f4")[2 * 62 + 54]
    assert v == rec[2, 54]
    back = read_ply(p)
    assert list(back) == names
    assert all(np.array_equal(back[nm], rec[:, i]) for i, nm in enumerate(names))


def test_checkpoint_round_trip(tmp_path):
    g = _cloud(1000, seed=9)
    path = tmp_path / "ck" / "epoch_1.pt"
    save_weights(g, path)
    state = torch.load(path, map_location="cpu", weights_only=True)
    assert set(state) == {"mu", "q", "s", "alpha", "A", "k_j", "N"} and state["N"] == 1000
    h = load_gaussians(path, "cpu")
    for k in ("mu", "q", "s", "alpha", "A", "k_j"):
        got = getattr(h, k)
        assert got.dtype == torch.float32 and got.is_contiguous()
        assert torch.equal(got, getattr(g, k))
