"""The reference's GPU kernel entry points on the HIP library.

Drop-in for ``tang0389/himuon`` ``src/himuon/triton_kernels`` (``XXT``,
``ba_plus_cAA``, ``fused_bmm_add``; triton_kernels/__init__.py:1-27): the
same call signatures and results (bf16 operands, fp32 accumulation, one bf16
rounding per product; fused_bmm_add rounds B @ X before adding a * X,
fused_bmm_add.py:73-88), computed by himuon_xxt / himuon_ba_plus_caa /
himuon_bmm_add. Dimensions that are not multiples of 128 are zero padded
(exact for all three products) into scratch tensors and sliced back. There is
no CPU path: non-HIP tensors raise, as the reference's stubs do without a GPU
(triton_kernels/__init__.py:8-19).
"""

from __future__ import annotations

import torch

from . import _native as nat

__all__ = ("XXT", "ba_plus_cAA", "fused_bmm_add")


def _check_bf16(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name}: HIP kernels need device tensors (no CPU path)")
    if t.dtype != torch.bfloat16:
        raise TypeError(f"{name}: bfloat16 tensors expected, got {t.dtype}")


def _padded(t: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """(B, r, c) -> contiguous (B, rows, cols) with zero padding (or t itself)."""
    if t.shape[-2:] == (rows, cols) and t.is_contiguous():
        return t
    out = torch.zeros((t.shape[0], rows, cols), device=t.device, dtype=t.dtype)
    out[:, : t.shape[-2], : t.shape[-1]] = t
    return out


def _r(n: int) -> int:
    return nat.round_up(n, nat.NS_ALIGN)


def _as3d(t: torch.Tensor) -> torch.Tensor:
    return t.unsqueeze(0) if t.ndim == 2 else t


def XXT(A: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = A @ A.T (XXT.py:76-104); A (..., M, K), out (..., M, M)."""
    assert A.ndim in (2, 3)
    M, K = A.shape[-2:]
    assert out.shape[-2:] == (M, M), "Output matrix has incorrect shape"
    _check_bf16("XXT", A)
    _check_bf16("XXT", out)
    a3 = _as3d(A)
    B = a3.shape[0]
    mp, kp = _r(M), _r(K)
    x = _padded(a3, mp, kp)
    o = torch.empty((B, mp, mp), device=A.device, dtype=A.dtype)
    nat.xxt(x, o, B, mp, kp)
    _as3d(out).copy_(o[:, :M, :M])
    return out


def ba_plus_cAA(A: torch.Tensor, alpha: float, beta: float, out: torch.Tensor) -> torch.Tensor:
    """out = alpha * A @ A.T + beta * A (ba_plus_cAA.py:90-120); A square."""
    assert A.ndim in (2, 3)
    M, K = A.shape[-2:]
    assert M == K, "Input matrix must be square"
    assert out.shape[-2:] == (M, M)
    _check_bf16("ba_plus_cAA", A)
    _check_bf16("ba_plus_cAA", out)
    a3 = _as3d(A)
    B = a3.shape[0]
    mp = _r(M)
    x = _padded(a3, mp, mp)
    o = torch.empty((B, mp, mp), device=A.device, dtype=A.dtype)
    nat.ba_plus_caa(x, o, B, mp, float(alpha), float(beta))
    _as3d(out).copy_(o[:, :M, :M])
    return out


def fused_bmm_add(B: torch.Tensor, X: torch.Tensor, a: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = B @ X + a * X with B @ X rounded to bf16 first (fused_bmm_add.py:98-135);
    B (Batch, M, M), X (Batch, M, N)."""
    Batch, M, K = B.shape
    _, _, N = X.shape
    assert M == K, "fused_bmm_add requires M == K for epilogue B@X + a*X"
    _check_bf16("fused_bmm_add", B)
    _check_bf16("fused_bmm_add", X)
    if out is None:
        out = torch.empty_like(X)
    mp, npd = _r(M), _r(N)
    b = _padded(B, mp, mp)
    x = _padded(X, mp, npd)
    o = torch.empty((Batch, mp, npd), device=X.device, dtype=X.dtype)
    nat.bmm_add(b, x, o, Batch, mp, npd, float(a))
    out.copy_(o[:, :M, :N])
    return out
