"""Torch-on-GPU references used by the GPU parity tests (not collected).

* ``ns5_torch_staged``: the reference's NS5 evaluated eagerly with torch in
  the dtypes of its GPU kernels — bf16 operands, fp32 accumulation, one bf16
  rounding per GEMM stage (XXT.py:62-63, ba_plus_cAA.py:78-85,
  fused_bmm_add.py:73-88, ns5_smem.py:84-101).
* ``ns5_torch_eager``: the reference test's pure-torch oracle
  (tests/integration/test_kernels.py:176-198): every torch op rounds to bf16.

bf16 batched products take contiguous operands only (a transposed view as the
right operand of a bf16 bmm is avoided on this platform).
"""

from __future__ import annotations

import numpy as np
import torch

A, B, C = 3.4445, -4.7750, 2.0315
EPS = 1e-7


def _bmm(x, y):
    return torch.bmm(x.contiguous(), y.contiguous())


def _t(x):
    return x.transpose(-2, -1).contiguous()


def ns5_torch_staged(G: torch.Tensor, steps: int = 5, round_once: bool = False) -> torch.Tensor:
    """round_once: the reference's 2-D third product, torch.addmm(X, B, X,
    beta=a) per matrix (himuon.py:249-253), instead of the batched
    fused_bmm_add form."""
    shape, dtype = G.shape, G.dtype
    X = G.reshape(-1, shape[-2], shape[-1]).to(torch.bfloat16)
    tall = shape[-2] > shape[-1]
    if tall:
        X = _t(X)
    xf = X.float()
    inv = 1.0 / (xf.square().sum(dim=(-2, -1), keepdim=True).sqrt() + EPS)
    X = (xf * inv).to(torch.bfloat16)
    for _ in range(steps):
        Am = _bmm(X, _t(X))  # bf16 out, fp32 accumulate
        Bm = torch.baddbmm(Am, Am, _t(Am), beta=B, alpha=C)  # fp32 epilogue, one rounding
        if round_once:
            X = torch.stack([torch.addmm(X[i], Bm[i], X[i], beta=A, alpha=1.0) for i in range(X.shape[0])])
        else:
            BX = _bmm(Bm, X)
            X = torch.add(BX, X, alpha=A)  # bf16(float(BX) + a * float(X))
    if tall:
        X = _t(X)
    return X.reshape(shape).to(dtype)


def ns5_torch_eager(G: torch.Tensor, steps: int = 5) -> torch.Tensor:
    shape, dtype = G.shape, G.dtype
    X = G.reshape(-1, shape[-2], shape[-1]).to(torch.bfloat16)
    tall = shape[-2] > shape[-1]
    if tall:
        X = _t(X)
    X = X / (X.norm(dim=(-2, -1), keepdim=True) + EPS)
    for _ in range(steps):
        Am = _bmm(X, _t(X))
        Bm = B * Am + C * _bmm(Am, Am)
        X = A * X + _bmm(Bm, X)
    if tall:
        X = _t(X)
    return X.reshape(shape).to(dtype)


def per_tile_rel_fro(out: torch.Tensor, ref: torch.Tensor) -> np.ndarray:
    """||out_t - ref_t||_F / ||ref_t||_F for each matrix of a (..., M, N) batch."""
    o = out.reshape(-1, out.shape[-2], out.shape[-1]).double()
    r = ref.reshape(-1, ref.shape[-2], ref.shape[-1]).double()
    num = (o - r).flatten(1).norm(dim=1)
    den = r.flatten(1).norm(dim=1).clamp_min(1e-30)
    return (num / den).cpu().numpy()


def well_conditioned(shape, dtype, seed=0, device="cuda") -> torch.Tensor:
    """Random matrices with singular values spread over [0.8, 1.2]
    (test_kernels.py:201-215), generated on the CPU from a seed."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g, dtype=torch.float64)
    U, _, Vh = torch.linalg.svd(x, full_matrices=False)
    k = U.shape[-1]
    s = torch.linspace(0.8, 1.2, k, dtype=torch.float64)
    return ((U * s.unsqueeze(-2)) @ Vh).to(dtype).to(device)
