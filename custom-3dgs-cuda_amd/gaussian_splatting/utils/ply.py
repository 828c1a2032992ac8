"""The Inria 3DGS ``point_cloud.ply`` export, counterpart of the reference's
scripts/run.py:66-170 (``save_ply`` / ``export_attributes``: same arguments,
attribute names and order, values), with the vertex records assembled on the
device by one HIP kernel (``custom_rasterizer_cuda.ply_records``) and written
with one copy to the host.  Viewers (SuperSplat, SIBR) read pre-activation
parameters: opacity logits, log-scales, unit quaternions (w, x, y, z), SH rest
coefficients channel-major.

The file is binary little-endian PLY 1.0 (the reference writes it with plyfile's
defaults): the header ``ply``, ``format binary_little_endian 1.0``, ``element
vertex N``, one ``property float <name>`` line per attribute, ``end_header``,
each line ended by a newline; then N records of float32.  ``read_ply`` parses
such a file back (any binary little-endian float vertex element)."""

from __future__ import annotations

import importlib
from pathlib import Path

import numpy as np
import torch as t

from gaussian_splatting.scene.gaussian import gaussian

_glue = importlib.import_module("gaussian_splatting.rasterizer.rasterize")


def _crc():
    if _glue.crc is None:
        raise ImportError("custom_rasterizer_cuda is not built. "
                          "Build it with: python custom-3dgs-cuda_amd/build.py")
    return _glue.crc


def attribute_names(n_rest: int) -> list[str]:
    """The Inria record's attribute names for ``n_rest`` rest coefficients per
    channel (run.py:125-136)."""
    return (["x", "y", "z", "nx", "ny", "nz"] + [f"f_dc_{i}" for i in range(3)]
            + [f"f_rest_{i}" for i in range(3 * n_rest)] + ["opacity"]
            + [f"scale_{i}" for i in range(3)] + [f"rot_{i}" for i in range(4)])


def ply_header(n: int, names: list[str]) -> bytes:
    lines = ["ply", "format binary_little_endian 1.0", f"element vertex {n}"]
    lines += [f"property float {nm}" for nm in names]
    lines.append("end_header")
    return ("\n".join(lines) + "\n").encode("ascii")


def vertex_records(gaussians: gaussian, max_sh_degree: int = 3) -> t.Tensor:
    """[N, 17 + 3K] float32 records on the Gaussians' device (K = (d + 1)^2 - 1)."""
    n_rest = (max_sh_degree + 1) ** 2 - 1
    with t.no_grad():
        mu = gaussians.mu.detach().float().contiguous()
        n = int(mu.shape[0])
        rest = gaussians.k_j.detach().float()
        if rest.ndim != 3 or rest.shape[-1] != 3:
            raise ValueError(f"Expected k_j shape (N, K, 3), got {tuple(rest.shape)}")
        if rest.shape[1] < n_rest:  # run.py:101-105: pad with zeros / truncate
            rest = t.cat([rest, rest.new_zeros(n, n_rest - rest.shape[1], 3)], dim=1)
        elif rest.shape[1] > n_rest:
            rest = rest[:, :n_rest, :]
        alpha = gaussians.alpha.detach().float().reshape(n).contiguous()
        # run.py:110-118: a checkpoint of probabilities (all in (0, 1), min > 1e-6)
        legacy = bool(((alpha > 0.0) & (alpha < 1.0)).all()) and float(alpha.min()) > 1e-6 \
            if n > 0 else False
        return _crc().ply_records(mu, gaussians.q.detach().float().contiguous(),
                                  gaussians.s.detach().float().contiguous(), alpha,
                                  gaussians.A.detach().float().reshape(n, 3).contiguous(),
                                  rest.contiguous(), legacy)


def save_ply(gaussians: gaussian, out_path, *, max_sh_degree: int = 3) -> None:
    """Export Gaussians as an official Inria 3DGS ``point_cloud.ply`` (run.py:66-165)."""
    out_path = Path(out_path)
    out_path.parent.mkdir(parents=True, exist_ok=True)
    n_rest = (max_sh_degree + 1) ** 2 - 1
    rec = vertex_records(gaussians, max_sh_degree).cpu().numpy()
    n = rec.shape[0]
    with open(out_path, "wb") as f:
        f.write(ply_header(n, attribute_names(n_rest)))
        f.write(np.ascontiguousarray(rec, dtype="<f4").tobytes())
    print(f"[export] Wrote {n} Gaussians (SH degree {max_sh_degree}, f_rest={3 * n_rest}) "
          f"-> {out_path}")


def export_attributes(gaussians: gaussian, out_path) -> None:
    """Backward-compatible alias for :func:`save_ply` (run.py:168-170)."""
    save_ply(gaussians, out_path)


def read_ply(path) -> dict:
    """The vertex element of a binary little-endian PLY of float properties:
    {name: float32 array [N]} in file order."""
    data = Path(path).read_bytes()
    end = data.index(b"end_header\n") + len(b"end_header\n")
    lines = data[:end].decode("ascii").splitlines()
    if lines[0] != "ply" or lines[1] != "format binary_little_endian 1.0":
        raise ValueError("not a binary little-endian PLY file")
    n, names = None, []
    for ln in lines[2:]:
        parts = ln.split()
        if parts[0] == "element":
            if parts[1] != "vertex":
                raise ValueError(f"unexpected element {parts[1]}")
            n = int(parts[2])
        elif parts[0] == "property":
            if parts[1] != "float":
                raise ValueError(f"unsupported property type {parts[1]}")
            names.append(parts[2])
    rec = np.frombuffer(data, dtype="<f4", count=n * len(names), offset=end)
    rec = rec.reshape(n, len(names))
    return {nm: rec[:, i].copy() for i, nm in enumerate(names)}
