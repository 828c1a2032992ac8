"""GPU parity of the PLY export (scripts/run.py:66-165 of the reference): the
records packed by the HIP kernel and written by save_ply, read back from the
file, against the record oracle (oracle/ply_oracle.py, pinned in test_ply.py):
bit for bit, except a legacy checkpoint's opacity logits (log of a
probability), within 1 ulp."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gaussian_splatting.utils.ply import attribute_names, read_ply, save_ply, vertex_records
from oracle import ply_oracle as po
from test_ply import _cloud

pytestmark = pytest.mark.gpu


def _to(g, device):
    for k in ("mu", "q", "s", "alpha", "A", "k_j"):
        setattr(g, k, getattr(g, k).to(device))
    return g


@pytest.mark.parametrize("n,legacy,deg,K", [(100_003, False, 3, 15), (50_001, True, 3, 15),
                                            (777, False, 1, 15), (64, False, 4, 15),
                                            (65, True, 3, 8), (1, False, 3, 15)])
def test_save_ply_matches_the_oracle(device, tmp_path, n, legacy, deg, K):
    g = _cloud(n, seed=n, legacy=legacy, K=K)
    want = po.vertex_records(g.mu, g.q, g.s, g.alpha, g.A, g.k_j, deg)
    _to(g, device)
    path = tmp_path / "point_cloud.ply"
    save_ply(g, path, max_sh_degree=deg)
    back = read_ply(path)
    names = attribute_names((deg + 1) ** 2 - 1)
    assert list(back) == names
    got = np.stack([back[nm] for nm in names], axis=1)
    op = names.index("opacity")
    cols = [i for i in range(len(names)) if i != op]
    assert np.array_equal(got[:, cols].view(np.uint32), want[:, cols].view(np.uint32))
    d = np.abs(got[:, op].view(np.int32).astype(np.int64) - want[:, op].view(np.int32))
    assert d.max() <= (1 if legacy else 0)


def test_vertex_records_stay_on_the_device(device):
    g = _to(_cloud(1000, seed=2), device)
    rec = vertex_records(g)
    assert rec.device.type == "cuda" and rec.shape == (1000, 62) and rec.dtype == torch.float32
