"""torch-CPU restatement of the reference's eager HiMuon step — TEST
INFRASTRUCTURE AND CPU BASELINE ONLY.

Only tests/ and the ``cpu_baseline`` leg of bench.py import it (as a checker
and as the reported CPU baseline); the product path (himuon_amd) never does.

The step of one Muon parameter as the reference writes it in torch ops
(tang0389/himuon, src/himuon/optimizers/himuon.py), on host tensors:

  momentum_       himuon.py:350-357: buf.mul_(mu).add_(g); Nesterov
                  e = g.add(buf, alpha=mu)
  tiles / untile  himuon.py:288-310 (_tile/_untile: zero pad, tile_h x tile_w
                  blocks, tall blocks transposed for NS), 704-719, 315-329
  newton_schulz   himuon.py:232-262 with the three products at the reference
                  kernels' rounding points, as torch bf16 ops: A = bmm(X, X^T)
                  (XXT.py:55-75), B = baddbmm(A, A, A^T, beta=b, alpha=c)
                  (ba_plus_cAA.py:58-85), X = bf16(bf16(bmm(B, X)) + a X)
                  with a X in fp32 (fused_bmm_add.py:65-88); for a 2-D input the third product
                  is addmm(X, B, X, beta=a) (himuon.py:249-253). X0 =
                  bf16(x / (||x||_F + eps)) with the norm in fp32 (:239-242).
  step_param      momentum, NS (tiled or, for numel <= tile area, the full
                  matrix), the lr scale (himuon.py:181-186) applied to the
                  update in the grad dtype (:257, 338-341), then WD and LR
                  (:215-228 / 333-348: p.mul_(1 - lr wd); p.add_(u, alpha=-lr)).

The GEMMs run in bf16 on the host's native bf16 units (torch / oneDNN): fp32
accumulation and one bf16 rounding per product, as on the GPU, but in the CPU
library's own summation order. NS outputs therefore agree with
himuon_oracle.ns5_staged to within bf16 rounding, not bit for bit; the
momentum, tiling, untiling and WD/LR agree exactly (pinned in
tests/test_torch_cpu_step.py).
"""

from __future__ import annotations

import math

import torch

NS_A, NS_B, NS_C = 3.4445, -4.7750, 2.0315
NS_EPS = 1e-7


def momentum_(g: torch.Tensor, buf: torch.Tensor, mu: float, nesterov: bool) -> torch.Tensor:
    """In-place momentum buffer update; returns the NS input (himuon.py:350-357)."""
    buf.mul_(mu).add_(g)
    return g.add(buf, alpha=mu) if nesterov else buf


def tiles(x: torch.Tensor, th: int, tw: int) -> torch.Tensor:
    """(R*C, m, n) NS operands of an (h, w) matrix, m <= n (tall blocks
    transposed), zero padded at the bottom/right edge."""
    h, w = x.shape
    R, C = -(-h // th), -(-w // tw)
    xp = torch.nn.functional.pad(x, (0, C * tw - w, 0, R * th - h))
    t = xp.reshape(R, th, C, tw).permute(0, 2, 1, 3).reshape(R * C, th, tw)
    return t.transpose(1, 2) if th > tw else t


def untile(t: torch.Tensor, h: int, w: int, th: int, tw: int) -> torch.Tensor:
    if th > tw:
        t = t.transpose(1, 2)
    R, C = -(-h // th), -(-w // tw)
    return t.reshape(R, C, th, tw).permute(0, 2, 1, 3).reshape(R * th, C * tw)[:h, :w]


def newton_schulz(G: torch.Tensor, steps: int = 5, eps: float = NS_EPS) -> torch.Tensor:
    """Quintic NS in bf16 GEMMs; (..., m, n) -> bf16, same shape. A 2-D input
    takes the 2-D third product (one rounding of B X + a X)."""
    a, b, c = NS_A, NS_B, NS_C
    X = G.to(torch.bfloat16)
    tall = X.shape[-2] > X.shape[-1]
    if tall:
        X = X.transpose(-2, -1)
    nrm = X.float().square().sum(dim=(-2, -1), keepdim=True).sqrt()
    X = (X.float() * (1.0 / (nrm + eps))).to(torch.bfloat16)
    two_d = X.dim() == 2
    if two_d:
        X = X.unsqueeze(0)
    X = X.contiguous()
    for _ in range(steps):
        Xt = X.transpose(1, 2).contiguous()
        A = torch.bmm(X, Xt)
        B = torch.baddbmm(A, A, A.transpose(1, 2).contiguous(), beta=b, alpha=c)
        if two_d:
            X = torch.addmm(X[0], B[0], X[0], beta=a).unsqueeze(0)
        else:  # a X in fp32: torch's CPU add(alpha=) on bf16 tensors rounds alpha to bf16
            X = (torch.bmm(B, X).float() + a * X.float()).to(torch.bfloat16)
    X = X[0] if two_d else X
    return X.transpose(-2, -1) if tall else X


def lr_scale(th: int, tw: int) -> float:
    """himuon.py:181-186 (lr_adjust 'tile'): 0.2 sqrt(max(rows, cols)) of the NS block."""
    return 0.2 * math.sqrt(max(th, tw))


def step_param(p: torch.Tensor, g: torch.Tensor, buf: torch.Tensor, lr: float, wd: float, tile: int,
               mu: float = 0.95, nesterov: bool = True, steps: int = 5) -> torch.Tensor:
    """One HiMuon step of one parameter, in place on p and buf; returns the
    update (grad dtype)."""
    e = momentum_(g, buf, mu, nesterov)
    h, w = e.shape
    if h * w <= tile * tile:
        th, tw = h, w
        u = newton_schulz(e, steps)
    else:
        th, tw = tile, tile
        u = untile(newton_schulz(tiles(e, th, tw), steps), h, w, th, tw)
    upd = u.to(g.dtype).mul_(lr_scale(th, tw))
    p.mul_(1.0 - lr * wd)
    p.add_(upd, alpha=-lr)
    return upd
