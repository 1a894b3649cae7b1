"""The reference's GPU kernel entry points on the HIP library.

Drop-in for ``tang0389/himuon`` ``src/himuon/triton_kernels``
(triton_kernels/__init__.py:1-27): ``XXT``, ``ba_plus_cAA``,
``fused_bmm_add`` and ``ns5_smem`` with the reference's call signatures.

* Operands may be bf16, fp16, fp32 or fp8 e5m2 (``fused_bmm_add``: both of one
  dtype); the result takes the dtype of ``out`` (fp32, bf16 or fp16), cast from
  an fp32 accumulator as the reference's ``tl.dot`` kernels do (XXT.py:62-63,
  ba_plus_cAA.py:65-85, fused_bmm_add.py:73-88). ``fused_bmm_add`` rounds
  ``B @ X`` to the output dtype before adding ``a * X``.
* bf16 operands with a bf16 output run the kernels of the optimizer's NS path
  (himuon_xxt / himuon_ba_plus_caa / himuon_bmm_add: bit-identical to torch's
  bf16 products); every other dtype pair runs the typed kernels
  (himuon_*_typed: fp16 MFMAs for fp16 and e5m2 operands, the e5m2 values
  widened exactly; three bf16 MFMAs per product for fp32 operands, 16
  significant bits of each, where the reference's fp32 dot uses TF32).
* ``ns5_smem`` (ns5_smem.py:195-263): bf16 only, M <= N, contiguous, a fresh
  tensor, always 5 iterations, the batched rounding of the third product. Its
  ``persistent`` / ``grid_size`` arguments choose the reference's Triton
  launch grid for ablations; here they are validated and accepted, and the
  library's own launch shape runs (one workgroup per tile on the LDS-resident
  kernel for 128-row tiles). ``ns5_smem_kernel``, a Triton kernel handle, has
  no counterpart.

Dimensions that are not multiples of 128 are zero padded (exact for all three
products) into scratch tensors and sliced back. There is no CPU path: non-HIP
tensors raise, as the reference's stubs do without a GPU
(triton_kernels/__init__.py:8-19).
"""

from __future__ import annotations

import torch

from . import _native as nat
from .engine import newton_schulz as _newton_schulz

__all__ = ("XXT", "ba_plus_cAA", "fused_bmm_add", "ns5_smem")

_OUT_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def _check_operand(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name}: HIP kernels need device tensors (no CPU path)")
    if t.dtype not in nat.PRODUCT_IN_CODES:
        raise TypeError(f"{name}: operands of {sorted(map(str, nat.PRODUCT_IN_CODES))} expected, got {t.dtype}")


def _check_out(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name}: HIP kernels need device tensors (no CPU path)")
    if t.dtype not in _OUT_DTYPES:
        raise TypeError(f"{name}: output of float32/bfloat16/float16 expected, got {t.dtype}")


def _bytes_view(t: torch.Tensor) -> torch.Tensor:
    """fp8 tensors as uint8 (zero-fill and copies on the raw bytes: byte 0 is +0)."""
    return t.view(torch.uint8) if t.element_size() == 1 else t


def _padded(t: torch.Tensor, rows: int, cols: int) -> torch.Tensor:
    """(B, r, c) -> contiguous (B, rows, cols) with zero padding (or t itself)."""
    if t.shape[-2:] == (rows, cols) and t.is_contiguous():
        return t
    out = torch.zeros((t.shape[0], rows, cols), device=t.device, dtype=t.dtype)
    _bytes_view(out)[:, : t.shape[-2], : t.shape[-1]] = _bytes_view(t)
    return out


def _r(n: int) -> int:
    return nat.round_up(n, nat.NS_ALIGN)


def _as3d(t: torch.Tensor) -> torch.Tensor:
    return t.unsqueeze(0) if t.ndim == 2 else t


def _native_bf16(*ts: torch.Tensor) -> bool:
    return all(t.dtype == torch.bfloat16 for t in ts)


def XXT(A: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """out = A @ A.T (XXT.py:76-104); A (..., M, K), out (..., M, M)."""
    assert A.ndim in (2, 3)
    M, K = A.shape[-2:]
    assert out.shape[-2:] == (M, M), "Output matrix has incorrect shape"
    _check_operand("XXT", A)
    _check_out("XXT", out)
    a3 = _as3d(A)
    B = a3.shape[0]
    mp, kp = _r(M), _r(K)
    x = _padded(a3, mp, kp)
    o = torch.empty((B, mp, mp), device=A.device, dtype=out.dtype)
    if _native_bf16(A, out):
        nat.xxt(x, o, B, mp, kp)
    else:
        nat.xxt_typed(x, o, B, mp, kp)
    _as3d(out).copy_(o[:, :M, :M])
    return out


def ba_plus_cAA(A: torch.Tensor, alpha: float, beta: float, out: torch.Tensor) -> torch.Tensor:
    """out = alpha * A @ A.T + beta * A (ba_plus_cAA.py:90-120); A square (and,
    as the reference's mirrored store assumes, symmetric)."""
    assert A.ndim in (2, 3)
    M, K = A.shape[-2:]
    assert M == K, "Input matrix must be square"
    assert out.shape[-2:] == (M, M)
    _check_operand("ba_plus_cAA", A)
    _check_out("ba_plus_cAA", out)
    a3 = _as3d(A)
    B = a3.shape[0]
    mp = _r(M)
    x = _padded(a3, mp, mp)
    o = torch.empty((B, mp, mp), device=A.device, dtype=out.dtype)
    if _native_bf16(A, out):
        nat.ba_plus_caa(x, o, B, mp, float(alpha), float(beta))
    else:
        nat.ba_plus_caa_typed(x, o, B, mp, float(alpha), float(beta))
    _as3d(out).copy_(o[:, :M, :M])
    return out


def fused_bmm_add(B: torch.Tensor, X: torch.Tensor, a: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """out = B @ X + a * X with B @ X rounded to the output dtype first
    (fused_bmm_add.py:98-135); B (Batch, M, M), X (Batch, M, N); out defaults
    to X's shape and dtype."""
    Batch, M, K = B.shape
    _, _, N = X.shape
    assert M == K, "fused_bmm_add requires M == K for epilogue B@X + a*X"
    _check_operand("fused_bmm_add", B)
    _check_operand("fused_bmm_add", X)
    if B.dtype != X.dtype:
        raise TypeError(f"fused_bmm_add: B and X of one dtype expected, got {B.dtype} and {X.dtype}")
    if out is None:
        if X.dtype not in _OUT_DTYPES:
            raise TypeError(f"fused_bmm_add: pass `out` (float32/bfloat16/float16) for {X.dtype} operands")
        out = torch.empty_like(X)
    _check_out("fused_bmm_add", out)
    mp, npd = _r(M), _r(N)
    b = _padded(B, mp, mp)
    x = _padded(X, mp, npd)
    o = torch.empty((Batch, mp, npd), device=X.device, dtype=out.dtype)
    if _native_bf16(B, X, out):
        nat.bmm_add(b, x, o, Batch, mp, npd, float(a))
    else:
        nat.bmm_add_typed(b, x, o, Batch, mp, npd, float(a))
    out.copy_(o[:, :M, :N])
    return out


def ns5_smem(X: torch.Tensor, *, persistent: bool = False, grid_size: int | None = None) -> torch.Tensor:
    """Fused 5-iteration NS on (B, M, N) or (M, N) bf16 tiles with M <= N
    (ns5_smem.py:195-263); returns a fresh tensor of X's shape. ``persistent``
    and ``grid_size`` are accepted for the reference's ablation calls
    (exp_ns5_rect_bench.py:178-179); the launch shape is the library's own."""
    assert X.ndim in (2, 3), f"ns5_smem expects 2D or 3D, got {X.ndim}D"
    M, N = X.shape[-2:]
    assert M <= N, f"ns5_smem expects M ≤ N, got ({M}, {N})"
    assert X.dtype == torch.bfloat16, f"ns5_smem is bf16-only, got {X.dtype}"
    assert X.is_contiguous(), "ns5_smem requires contiguous input"
    if grid_size is not None and (not isinstance(grid_size, int) or grid_size <= 0):
        raise ValueError(f"ns5_smem: grid_size must be a positive int, got {grid_size!r}")
    del persistent
    # a 2-D input runs as a batch of one, as the reference's kernel does
    # (batched rounding of the third product, not the 2-D addmm form)
    return _newton_schulz(_as3d(X), steps=5).view(X.shape)
