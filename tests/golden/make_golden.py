"""Generate the committed fixtures in tests/golden/golden.npz.

Every expected value here comes from an implementation independent of the
oracle function it pins:

* tile maps: a brute-force double loop over parameter elements, written from
  the reference's description of the concat-buffer layout (himuon.py:704-719:
  tile (r, c) of a zero-padded (h, w) parameter at index r*C + c);
* momentum: torch's own CPU ops, literally ``buf.mul_(mu).add_(g)`` and
  ``g.add(buf, alpha=mu)`` (himuon.py:354-356);
* NS5: the SVD closed form U f(S/||G||) V^T in float64 with f the quintic map
  iterated 5 times (muon.py:14-44; the iteration itself is not used).

Run: python tests/golden/make_golden.py   (writes golden.npz next to it)
"""

from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
A, B, C = 3.4445, -4.7750, 2.0315
EPS = 1e-7

TILE_CASES = [
    # (h, w, tile_h, tile_w)
    (40, 27, 16, 8),
    (27, 40, 8, 16),
    (33, 33, 16, 16),
    (32, 64, 16, 16),
    (7, 50, 4, 16),
]

NS_CASES = [
    # (seed, shape)
    (1, (3, 8, 12)),
    (2, (2, 12, 8)),
    (3, (16, 16)),
    (4, (1, 5, 40)),
]


def brute_tile_map(h, w, th, tw):
    R = -(-h // th)
    Cc = -(-w // tw)
    out = np.full((R * Cc, th, tw), -1, dtype=np.int64)
    for row in range(h):
        for col in range(w):
            r, i = divmod(row, th)
            c, j = divmod(col, tw)
            out[r * Cc + c, i, j] = row * w + col
    return out


def quintic_scalar(s):
    for _ in range(5):
        s = A * s + B * s**3 + C * s**5
    return s


def ns_svd(G):
    G = np.asarray(G, dtype=np.float64)
    U, S, Vt = np.linalg.svd(G, full_matrices=False)
    nrm = np.sqrt((G * G).sum(axis=(-2, -1)))
    f = quintic_scalar(S / (nrm[..., None] + EPS))
    return (U * f[..., None, :]) @ Vt


def main():
    out = {}
    for k, (h, w, th, tw) in enumerate(TILE_CASES):
        out[f"tilemap_{k}"] = brute_tile_map(h, w, th, tw)
        out[f"tilemap_{k}_args"] = np.array([h, w, th, tw], dtype=np.int64)

    g = torch.Generator().manual_seed(7)
    for dt_name, dt in (("float32", torch.float32), ("bfloat16", torch.bfloat16)):
        grad = (torch.randn(64, 48, generator=g) * 1e-3).to(dt)
        buf0 = (torch.randn(64, 48, generator=g) * 1e-3).to(dt)
        buf = buf0.clone()
        buf.mul_(0.95).add_(grad)
        geff = grad.add(buf, alpha=0.95)
        out[f"mom_{dt_name}_g"] = grad.float().numpy()
        out[f"mom_{dt_name}_buf0"] = buf0.float().numpy()
        out[f"mom_{dt_name}_buf1"] = buf.float().numpy()
        out[f"mom_{dt_name}_geff"] = geff.float().numpy()

    for k, (seed, shape) in enumerate(NS_CASES):
        rng = np.random.default_rng(seed)
        G = rng.standard_normal(shape)
        out[f"ns_{k}_in"] = G
        out[f"ns_{k}_out"] = ns_svd(G)

    np.savez_compressed(os.path.join(HERE, "golden.npz"), **out)
    print("wrote", os.path.join(HERE, "golden.npz"), len(out), "arrays")


if __name__ == "__main__":
    main()
