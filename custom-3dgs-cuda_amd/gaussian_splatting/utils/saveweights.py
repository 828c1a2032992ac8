"""Checkpoints, counterpart of the reference's gaussian_splatting/utils/saveweights.py:5-20
and the loader of scripts/run.py:55-63: the same ``.pt`` layout (a dict of CPU fp32
tensors mu, q, s, alpha, A, k_j and the count N), so checkpoints move between the
two builds unchanged."""

from __future__ import annotations

from pathlib import Path

import torch as t

from gaussian_splatting.scene.gaussian import gaussian

KEYS = ("mu", "q", "s", "alpha", "A", "k_j")


def save_weights(gaussians, path) -> None:
    """Save Gaussian parameters to a .pt checkpoint (saveweights.py:5-20)."""
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    state = {k: getattr(gaussians, k).detach().cpu() for k in KEYS}
    state["N"] = gaussians.N
    t.save(state, path)


def load_gaussians(checkpoint_path, device) -> gaussian:
    """A checkpoint back into a gaussian on ``device`` (run.py:55-63), read with
    ``weights_only=True``: fp32, contiguous."""
    state = t.load(checkpoint_path, map_location="cpu", weights_only=True)
    n = int(state["N"])
    g = gaussian(n)
    for k in KEYS:
        setattr(g, k, state[k].to(device=device, dtype=t.float32).contiguous())
    g.N = n
    return g
