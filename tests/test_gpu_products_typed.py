"""GPU parity of the reference's kernel entry points for every operand dtype
its own tests use (tests/integration/test_kernels.py:36-165): fp8 e5m2 and
fp16 operands with an fp16 result, fp16 and fp32 operands of fused_bmm_add
with the output dtype following ``out``, and ns5_smem (ns5_smem.py:195-263).

Each case runs through himuon_amd.kernels (the typed HIP kernels) and is
checked twice:
* with the reference test's own tolerance against the torch op it names;
* against an fp64 evaluation of the same mathematics on the CPU, with an
  error bound built from the reference kernel's rounding points (fp32
  accumulator cast to ``out``; fused_bmm_add rounds B @ X before adding
  a * X): one unit in the last place of the output dtype per rounding, plus
  the fp32 accumulation error 2 K 2^-24 times the sum of |terms| (16-bit and
  e5m2 operands: every product is exact in fp32), plus for fp32 operands
  (three bf16 MFMAs per product, 16 significant bits of each operand) 2^-15
  times the sum of |terms| -- tighter than the TF32 inputs (11 bits) of the
  reference's fp32 dot.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from himuon_amd import kernels as K
    from himuon_amd.engine import newton_schulz

    from gpu_ref import ns5_torch_staged

DEV = "cuda"
A_ = 3.4445
HAS_FP8 = hasattr(torch, "float8_e5m2")


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _mant(dtype) -> int:
    return {torch.float16: 10, torch.bfloat16: 7, torch.float32: 23}[dtype]


def _ulp(x: torch.Tensor, dtype) -> torch.Tensor:
    """Spacing of `dtype` at |x| (fp64 in and out; subnormal spacing below)."""
    info = torch.finfo(dtype)
    mag = x.abs().clamp_min(info.tiny)
    return torch.pow(2.0, torch.floor(torch.log2(mag)) - _mant(dtype))


def _assert_bounded(got, exact, terms, dtype, K, in_dtype, roundings=()):
    """|got - exact| <= ulp(dtype, exact) + ulp of each extra rounded
    intermediate + (2 K 2^-24 [+ 2^-15 for fp32 operands]) * terms."""
    g = got.double().cpu()
    bound = _ulp(exact, dtype) + terms * (2 * K * 2.0 ** -24 + (2.0 ** -15 if in_dtype == torch.float32 else 0.0))
    for r in roundings:
        bound = bound + _ulp(r, dtype)
    err = (g - exact).abs()
    assert bool((err <= bound).all()), (int((err > bound).sum()), float((err / bound).max()))


@pytest.mark.skipif(not HAS_FP8, reason="torch without float8_e5m2")
def test_xxt_fp8_e5m2_into_fp16():
    """test_kernels.py:50-66: small-integer e5m2 operands, fp16 output. The
    products of integers |a| <= 5 over K = 64 are integers below 2048, exact
    in fp16: the result equals the exact product bit for bit."""
    M, Kd = 128, 64
    A_float = torch.randint(-5, 5, (M, Kd), generator=_gen(1)).to(torch.float16).to(DEV)
    A = A_float.to(torch.float8_e5m2)
    out = torch.empty((M, M), device=DEV, dtype=torch.float16)
    K.XXT(A, out)
    ref = A_float @ A_float.T
    assert torch.allclose(out, ref, atol=0.5, rtol=1e-1)
    exact = A_float.double().cpu() @ A_float.double().cpu().T
    assert torch.equal(out.double().cpu(), exact)


@pytest.mark.skipif(not HAS_FP8, reason="torch without float8_e5m2")
@pytest.mark.parametrize("M", [128, 200, 384])
def test_ba_plus_caa_fp8_e5m2_into_fp16(M):
    """test_kernels.py:91-118: A = normalised (R R^T) cast to e5m2, fp16
    output; the reference test's 0.2 tolerance, and 1 ulp of fp16 against
    fp64 on the e5m2 values."""
    R = torch.randn((M, M), generator=_gen(M)).to(torch.float16).to(DEV)
    Af = R @ R.T
    Af = Af / (Af.norm() + 1e-6)
    A = Af.to(torch.float8_e5m2)
    A_ref = A.to(torch.float16)
    alpha, beta = 0.5, 0.3
    out = torch.empty((M, M), device=DEV, dtype=torch.float16)
    K.ba_plus_cAA(A, alpha, beta, out)
    assert torch.allclose(out, alpha * (A_ref @ A_ref.T) + beta * A_ref, atol=0.2, rtol=0.2)
    a64 = A_ref.double().cpu()
    exact = alpha * (a64 @ a64.T) + beta * a64
    terms = alpha * (a64.abs() @ a64.abs().T) + beta * a64.abs()
    _assert_bounded(out, exact, terms, torch.float16, M, torch.float16)
    assert torch.equal(out, out.T)  # mirrored store


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fused_bmm_add_dtype(dtype):
    """test_kernels.py:148-165: the output dtype follows `out`, with the
    reference test's tolerance against torch's ops in that dtype; and the fp64
    model of the reference kernel's rounding points."""
    Batch, M, N = 4, 128, 128
    g = _gen(0)
    B = torch.randn((Batch, M, M), generator=g).to(dtype).to(DEV)
    X = torch.randn((Batch, M, N), generator=g).to(dtype).to(DEV)
    out = torch.empty((Batch, M, N), device=DEV, dtype=dtype)
    got = K.fused_bmm_add(B, X, A_, out=out)
    assert got is out and got.dtype == dtype
    ref = torch.bmm(B, X) + A_ * X
    atol = 1e-1 if dtype != torch.float32 else 5e-2
    assert torch.allclose(got, ref, atol=atol, rtol=1e-2), (got.float() - ref.float()).abs().max()
    b64, x64 = B.double().cpu(), X.double().cpu()
    bx = torch.bmm(b64, x64)
    terms = torch.bmm(b64.abs(), x64.abs()) + abs(A_) * x64.abs()
    # out = dtype(dtype(B X) + a X): B X is rounded once more before the add
    _assert_bounded(got, bx + A_ * x64, terms, dtype, M, dtype,
                    roundings=() if dtype == torch.float32 else (bx,))


@pytest.mark.parametrize("in_dtype,out_dtype", [
    (torch.float32, torch.float32), (torch.float32, torch.bfloat16), (torch.float16, torch.float32),
    (torch.float16, torch.float16), (torch.bfloat16, torch.float32), (torch.bfloat16, torch.float16),
])
@pytest.mark.parametrize("shape", [(2, 128, 256), (3, 100, 70), (1, 384, 130)], ids=["aligned", "pad", "wide-pad"])
def test_xxt_and_ba_plus_caa_typed(in_dtype, out_dtype, shape):
    """XXT (M x K) and ba_plus_cAA (on the symmetric XXT result) for mixed
    dtype pairs, against fp64: fp32 operands within 1e-4 of the product scale
    and 1 ulp of a 16-bit output on top; 16-bit operands within 1 ulp of the
    output dtype (products exact in fp32)."""
    Bt, M, Kd = shape
    A = (torch.randn(shape, generator=_gen(M + Kd)) * 0.1).to(in_dtype).to(DEV)
    out = torch.empty((Bt, M, M), device=DEV, dtype=out_dtype)
    K.XXT(A, out)
    a64 = A.double().cpu()
    exact = torch.bmm(a64, a64.transpose(1, 2))
    terms = torch.bmm(a64.abs(), a64.abs().transpose(1, 2))
    _assert_bounded(out, exact, terms, out_dtype, Kd, in_dtype)
    assert torch.equal(out, out.transpose(1, 2))
    # ba_plus_cAA on a symmetric operand of the same dtype
    S = out.to(in_dtype) if out_dtype != in_dtype else out.clone()
    S = (S / S.double().abs().amax().clamp_min(1e-6).to(S.dtype)).to(in_dtype).contiguous()
    o2 = torch.empty((Bt, M, M), device=DEV, dtype=out_dtype)
    alpha, beta = 2.0315, -4.7750
    K.ba_plus_cAA(S, alpha, beta, o2)
    s64 = S.double().cpu()
    ex2 = alpha * torch.bmm(s64, s64.transpose(1, 2)) + beta * s64
    sc2 = abs(alpha) * torch.bmm(s64.abs(), s64.abs().transpose(1, 2)) + abs(beta) * s64.abs()
    _assert_bounded(o2, ex2, sc2, out_dtype, M, in_dtype)


@pytest.mark.parametrize("Batch,M,N", [(4, 100, 70), (2, 50, 130), (3, 200, 100)])
def test_fused_bmm_add_boundary_fp16(Batch, M, N):
    """test_kernels.py:117-140's unaligned dims with fp16 operands."""
    g = _gen(Batch * M + N)
    B = torch.randn((Batch, M, M), generator=g).to(torch.float16).to(DEV)
    X = torch.randn((Batch, M, N), generator=g).to(torch.float16).to(DEV)
    got = K.fused_bmm_add(B, X, A_)
    ref = torch.bmm(B, X) + A_ * X
    assert got.shape == X.shape and got.dtype == torch.float16
    assert torch.allclose(got, ref, atol=1e-1, rtol=1e-2), (got.float() - ref.float()).abs().max()


def test_typed_products_reject_mixed_and_bad_dtypes():
    B = torch.zeros((1, 128, 128), device=DEV, dtype=torch.float16)
    X = torch.zeros((1, 128, 128), device=DEV, dtype=torch.float32)
    with pytest.raises(TypeError):
        K.fused_bmm_add(B, X, 1.0)
    with pytest.raises(TypeError):
        K.XXT(torch.zeros((128, 64), device=DEV, dtype=torch.int32), torch.empty((128, 128), device=DEV))
    with pytest.raises(TypeError):
        K.XXT(torch.zeros((128, 64), device=DEV), torch.empty((128, 128), device=DEV, dtype=torch.float64))


@pytest.mark.parametrize("shape", [(4, 128, 512), (8, 128, 128), (2, 64, 256), (128, 128), (3, 32, 1024)],
                         ids=["128x512", "128x128", "64x256", "2d", "32x1024"])
def test_ns5_smem(shape):
    """ns5_smem(X) == the batched NS5 of torch in the same dtypes on the GPU,
    bit for bit (per-tile rel. Frobenius <= 1e-2 a fortiori), a fresh tensor,
    for every call form the reference's benchmarks use."""
    X = (torch.randn(shape, generator=_gen(sum(shape))) * 1e-3).to(torch.bfloat16).to(DEV)
    X_keep = X.clone()
    outs = [K.ns5_smem(X), K.ns5_smem(X, persistent=True), K.ns5_smem(X, grid_size=7)]
    ref = ns5_torch_staged(X.view(-1, *shape[-2:])).view(shape)
    for o in outs:
        assert o.shape == X.shape and o.dtype == torch.bfloat16 and o.data_ptr() != X.data_ptr()
        assert torch.equal(o, ref)
    assert torch.equal(X, X_keep)
    assert torch.equal(outs[0], newton_schulz(X.view(-1, *shape[-2:])).view(shape))


def test_ns5_smem_rejects_what_the_reference_rejects():
    with pytest.raises(AssertionError):
        K.ns5_smem(torch.zeros((2, 256, 128), device=DEV, dtype=torch.bfloat16))  # M > N
    with pytest.raises(AssertionError):
        K.ns5_smem(torch.zeros((2, 128, 128), device=DEV, dtype=torch.float32))  # bf16 only
    with pytest.raises(AssertionError):
        K.ns5_smem(torch.zeros((2, 128, 256), device=DEV, dtype=torch.bfloat16).transpose(1, 2).transpose(1, 2)[:, :, ::2])
    with pytest.raises(AssertionError):
        K.ns5_smem(torch.zeros((128,), device=DEV, dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        K.ns5_smem(torch.zeros((2, 128, 128), device=DEV, dtype=torch.bfloat16), grid_size=0)
