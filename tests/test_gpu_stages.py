"""GPU parity of the three NS products one at a time, in the manner of the
reference's building-block tests (tests/integration/test_kernels.py:36-172):
each product against the torch op it stands for, in the same dtypes on the
same GPU.

* XXT:            A = bf16(X X^T)               vs torch.bmm(X, X^T)
* ba_plus_cAA:    B = bf16(c A A^T + b A)       vs torch.baddbmm(A, A, A^T, beta=b, alpha=c)
* fused_bmm_add:  X' = bf16(bf16(B X) + a X)    vs torch.add(torch.bmm(B, X), X, alpha=a)
* 2-D form:       X' = bf16(B X + a X)          vs torch.addmm(X, B, X, beta=a)
* ba_bmm_add:     the last two fused (B on chip) vs the two stages, bit for bit

The kernels accumulate each output in one fp32 register over k in ascending
order with the same MFMA shape as torch's bf16 GEMMs on this GPU, so the
products are bit-identical to torch's; the Gram outputs are exactly
symmetric. Inputs come from CPU generators (seeded) and are copied over.
Shapes cover both kernel families (256-block stream kernels and 128-block
kernels) and the reference test's unaligned shapes (through the zero-padding
wrappers of himuon_amd.kernels, with the reference test's tolerances).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from himuon_amd import _native as nat
    from himuon_amd import kernels as K

DEV = "cuda"
A_, B_, C_ = 3.4445, -4.7750, 2.0315


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).to(DEV)


def _t(x):
    return x.transpose(-2, -1).contiguous()


def _normalised(x):
    """Tiles scaled to unit Frobenius norm, as NS feeds its products."""
    xf = x.float()
    return (xf / xf.flatten(1).norm(dim=1).view(-1, 1, 1)).to(torch.bfloat16)


def _sym(a):
    """A = bf16(X X^T) of a random X: the symmetric input GramB sees."""
    return torch.bmm(a, _t(a))


FAMILIES = ["auto", "block128"]
# (batch, M, K): M, K multiples of 128; 256-multiples run the stream kernels
GRAM_SHAPES = [(3, 256, 256), (2, 512, 512), (2, 256, 1024), (2, 1024, 1024), (3, 128, 384), (2, 384, 640)]
APPLY_SHAPES = [(3, 256, 256), (2, 512, 512), (2, 512, 1024), (2, 1024, 3072), (3, 128, 384), (2, 384, 640)]


@pytest.mark.parametrize("family", FAMILIES)
@pytest.mark.parametrize("batch,M,Kd", GRAM_SHAPES, ids=[f"{b}x{m}x{k}" for b, m, k in GRAM_SHAPES])
def test_xxt_bit_identical_to_torch_bmm(batch, M, Kd, family):
    print(f"[xxt] {batch}x{M}x{Kd} {family}", flush=True)
    x = _normalised(_rand((batch, M, Kd), seed=M + Kd))
    out = torch.full((batch, M, M), float("nan"), device=DEV, dtype=torch.bfloat16)
    nat.xxt(x, out, batch, M, Kd, family=family)
    ref = torch.bmm(x, _t(x))
    assert torch.equal(out, _t(out)), "XXT output not exactly symmetric"
    assert torch.equal(out, ref), f"max |diff| {(out.float() - ref.float()).abs().max().item()}"


@pytest.mark.parametrize("family", FAMILIES)
@pytest.mark.parametrize("batch,M,Kd", GRAM_SHAPES, ids=[f"{b}x{m}x{k}" for b, m, k in GRAM_SHAPES])
def test_ba_plus_caa_bit_identical_to_torch_baddbmm(batch, M, Kd, family):
    print(f"[ba_plus_caa] {batch}x{M} {family}", flush=True)
    A = _sym(_normalised(_rand((batch, M, Kd), seed=3 * M + Kd)))
    out = torch.full((batch, M, M), float("nan"), device=DEV, dtype=torch.bfloat16)
    nat.ba_plus_caa(A, out, batch, M, C_, B_, family=family)
    ref = torch.baddbmm(A, A, _t(A), beta=B_, alpha=C_)
    assert torch.equal(out, _t(out)), "ba_plus_cAA output not exactly symmetric"
    assert torch.equal(out, ref), f"max |diff| {(out.float() - ref.float()).abs().max().item()}"


@pytest.mark.parametrize("family", FAMILIES)
@pytest.mark.parametrize("batch,M,N", APPLY_SHAPES, ids=[f"{b}x{m}x{n}" for b, m, n in APPLY_SHAPES])
def test_bmm_add_bit_identical_to_torch(batch, M, N, family):
    print(f"[bmm_add] {batch}x{M}x{N} {family}", flush=True)
    X = _normalised(_rand((batch, M, N), seed=M + 7 * N))
    Bm = torch.baddbmm(_sym(X), _sym(X), _t(_sym(X)), beta=B_, alpha=C_)
    out = torch.full((batch, M, N), float("nan"), device=DEV, dtype=torch.bfloat16)
    nat.bmm_add(Bm, X, out, batch, M, N, A_, family=family)
    ref = torch.add(torch.bmm(Bm, X), X, alpha=A_)  # bf16(bf16(B X) + a X)
    assert torch.equal(out, ref), f"max |diff| {(out.float() - ref.float()).abs().max().item()}"


@pytest.mark.parametrize("family", FAMILIES)
@pytest.mark.parametrize("batch,M,N", APPLY_SHAPES[:4], ids=[f"{b}x{m}x{n}" for b, m, n in APPLY_SHAPES[:4]])
def test_bmm_add_2d_form_matches_torch_addmm(batch, M, N, family):
    """The reference's 2-D third product (himuon.py:252-253), one rounding."""
    print(f"[bmm_add 2d] {batch}x{M}x{N} {family}", flush=True)
    X = _normalised(_rand((batch, M, N), seed=M + 11 * N))
    Bm = torch.baddbmm(_sym(X), _sym(X), _t(_sym(X)), beta=B_, alpha=C_)
    out = torch.empty((batch, M, N), device=DEV, dtype=torch.bfloat16)
    nat.bmm_add(Bm, X, out, batch, M, N, A_, round_once=True, family=family)
    ref = torch.stack([torch.addmm(X[i], Bm[i], X[i], beta=A_, alpha=1.0) for i in range(batch)])
    diff = out != ref
    # torch.addmm's epilogue: alpha * acc + beta * C in fp32, then one rounding
    # to bf16; elements it rounds differently from fma(a, x, acc) are at most
    # one bf16 ulp apart and rare (fp32 rounding of a*x before the sum).
    n_diff = int(diff.sum())
    if n_diff:
        ulp = (out.float() - ref.float()).abs()[diff] / ref.float().abs()[diff].clamp_min(1e-30)
        print(f"  {n_diff} of {out.numel()} elements differ, max rel {ulp.max().item():.2e}", flush=True)
        assert n_diff <= out.numel() * 1e-3 and ulp.max().item() <= 2**-7
    # and it is not the batched form
    twice = torch.add(torch.bmm(Bm, X), X, alpha=A_)
    assert not torch.equal(out, twice)


@pytest.mark.parametrize("round_once", [False, True])
def test_fused_ba_bmm_add_equals_the_two_stages(round_once):
    """himuon_ba_bmm_add (B kept on chip) == ba_plus_cAA then fused_bmm_add,
    bit for bit, and == torch's baddbmm then bmm + add."""
    print(f"[ba_bmm_add] round_once={round_once}", flush=True)
    n = 6
    X = _normalised(_rand((n, 512, 512), seed=17))
    A = _sym(X)
    Bm = torch.empty_like(A)
    nat.ba_plus_caa(A, Bm, n, 512, C_, B_)
    two = torch.empty_like(X)
    nat.bmm_add(Bm, X, two, n, 512, 512, A_, round_once=round_once)
    fused = torch.full_like(X, float("nan"))
    nat.ba_bmm_add(A, X, fused, n, C_, B_, A_, round_once=round_once)
    assert torch.equal(fused, two)
    if not round_once:
        ref = torch.add(torch.bmm(torch.baddbmm(A, A, _t(A), beta=B_, alpha=C_), X), X, alpha=A_)
        assert torch.equal(fused, ref)


@pytest.mark.parametrize("n", [1, 3, 65, 257, 2049])
def test_fused_ba_bmm_add_tile_counts(n):
    """The fused kernel's persistent item walk (4 panels per tile, a
    contiguous item range per XCD, 32 workgroups per XCD) at tile counts that
    leave XCDs idle (1, 3), end ranges mid-tile and mid-walk (65, 257) and run
    up to 9 items per workgroup (2049): bit for bit the two-stage result, every
    tile written (the output starts as NaN)."""
    print(f"[ba_bmm_add] n={n}", flush=True)
    X = _normalised(_rand((n, 512, 512), seed=n))
    A = torch.empty_like(X)
    nat.xxt(X, A, n, 512, 512)
    Bm = torch.empty_like(A)
    nat.ba_plus_caa(A, Bm, n, 512, C_, B_)
    two = torch.empty_like(X)
    nat.bmm_add(Bm, X, two, n, 512, 512, A_)
    fused = torch.full_like(X, float("nan"))
    nat.ba_bmm_add(A, X, fused, n, C_, B_, A_)
    assert torch.equal(fused, two)


def test_stage_products_compose_to_ns_iteration():
    """One NS iteration as XXT -> ba_plus_cAA -> fused_bmm_add equals
    himuon_ns5 with steps = 1 on the same normalised tiles, bit for bit."""
    x = _normalised(_rand((4, 512, 512), seed=5, scale=1e-3))
    A = torch.empty(4, 512, 512, device=DEV, dtype=torch.bfloat16)
    Bm = torch.empty_like(A)
    X1 = torch.empty_like(x)
    nat.xxt(x, A, 4, 512, 512)
    nat.ba_plus_caa(A, Bm, 4, 512, C_, B_)
    nat.bmm_add(Bm, x, X1, 4, 512, 512, A_)
    tiles, alt = x.clone(), torch.empty_like(x)
    inv = torch.ones(4, device=DEV)
    ws = torch.empty(nat.ns5_workspace_bytes(4, 512, 512), device=DEV, dtype=torch.uint8)
    nat.ns5(tiles, alt, inv, 4, 512, 512, 1, ws, 4)
    assert torch.equal(alt, X1)


# -- the reference's kernel API (himuon_amd.kernels), reference test shapes ------
def test_reference_api_xxt_and_ba_plus_caa():
    """test_kernels.py:36-111 (bf16 cases) through the drop-in wrappers."""
    A = _rand((128, 64), seed=1)
    C = torch.empty((128, 128), device=DEV, dtype=torch.bfloat16)
    K.XXT(A, C)
    assert torch.allclose(C, A @ A.T, atol=1e-2, rtol=1e-2)
    assert torch.equal(C, C.T)
    Ar = _rand((128, 128), seed=2)
    S = Ar @ Ar.T
    alpha, beta = 0.5, 0.3
    out = torch.empty((128, 128), device=DEV, dtype=torch.bfloat16)
    K.ba_plus_cAA(S, alpha, beta, out)
    assert torch.allclose(out, alpha * (S @ S.T) + beta * S, atol=1e-2, rtol=1e-2)
    # batched, unaligned (zero padding in the wrapper)
    A3 = _rand((3, 100, 70), seed=3)
    C3 = torch.empty((3, 100, 100), device=DEV, dtype=torch.bfloat16)
    K.XXT(A3, C3)
    assert torch.allclose(C3, torch.bmm(A3, _t(A3)), atol=1e-2, rtol=1e-2)


@pytest.mark.parametrize("Batch,M,N", [(4, 100, 70), (2, 50, 130), (3, 200, 100), (4, 128, 128)])
def test_reference_api_fused_bmm_add_boundary(Batch, M, N):
    """test_kernels.py:117-140: unaligned dims, the reference test's tolerance."""
    torch.manual_seed(42)
    g = torch.Generator().manual_seed(Batch * M + N)
    B = torch.randn((Batch, M, M), generator=g).to(torch.bfloat16).to(DEV)
    X = torch.randn((Batch, M, N), generator=g).to(torch.bfloat16).to(DEV)
    got = K.fused_bmm_add(B, X, A_)
    ref = torch.bmm(B, X) + A_ * X
    assert got.shape == X.shape and got.dtype == X.dtype
    assert torch.allclose(got, ref, atol=1e-1, rtol=1e-2), (got.float() - ref.float()).abs().max()


def test_reference_api_rejects_host_tensors():
    A = torch.zeros((128, 64), dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        K.XXT(A, torch.empty((128, 128), dtype=torch.bfloat16))
