"""CPU restatement of the reference's PLY vertex records — TEST INFRASTRUCTURE
ONLY (tests/ use it as the checker; the product never imports it).

Follows scripts/run.py:66-165 of kmurungi/custom-3dgs-cuda (save_ply), in numpy
fp32 with the operations torch performs there on CPU tensors:
  f_dc = A; f_rest = k_j transposed to (N, 3, K) and flattened (channel-major,
  run.py:98-108), padded with zeros / truncated to K = (d + 1)^2 - 1;
  opacity = the stored logit, or for a checkpoint of probabilities (every value
  in (0, 1) and the least above 1e-6) log(a / (1 - a)) of a clamped to
  [1e-6, 1 - 1e-6] (run.py:110-118; the log rounded from float64);
  scale = the log-scales; rot = q / max(|q|, 1e-8) with |q| the square root of
  the squares summed in order in fp32 (torch's CPU norm over the last
  dimension, measured), normals 0.
plyfile (the reference's writer) is absent here; the file layout is pinned by the
PLY specification in tests/test_ply.py."""

from __future__ import annotations

import numpy as np


def vertex_records(mu, q, s, alpha, A, k_j, max_sh_degree: int = 3) -> np.ndarray:
    f = np.float32
    mu, q, s, A = (np.asarray(a, f) for a in (mu, q, s, A))
    n = mu.shape[0]
    rest = np.asarray(k_j, f).reshape(n, -1, 3)
    K = (max_sh_degree + 1) ** 2 - 1
    if rest.shape[1] < K:
        rest = np.concatenate([rest, np.zeros((n, K - rest.shape[1], 3), f)], axis=1)
    rest = rest[:, :K, :]
    f_rest = rest.transpose(0, 2, 1).reshape(n, 3 * K)
    a = np.asarray(alpha, f).reshape(n, 1)
    if n and np.all((a > 0) & (a < 1)) and float(a.min()) > 1e-6:
        ac = np.clip(a, f(1e-6), f(1.0 - 1e-6))
        opacity = np.log((ac / (f(1.0) - ac)).astype(np.float64)).astype(f)
    else:
        opacity = a
    qq = q.reshape(n, 4)
    n2 = (((qq[:, 0] * qq[:, 0] + qq[:, 1] * qq[:, 1]) + qq[:, 2] * qq[:, 2])
          + qq[:, 3] * qq[:, 3]).astype(f)
    norm = np.maximum(np.sqrt(n2).astype(f), f(1e-8)).reshape(n, 1)
    rot = (qq / norm).astype(f)
    return np.concatenate([mu, np.zeros((n, 3), f), A.reshape(n, 3), f_rest, opacity,
                           s.reshape(n, 3), rot], axis=1).astype(f)
