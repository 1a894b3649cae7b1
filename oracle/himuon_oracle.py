"""CPU oracle for the HiMuon step — TEST INFRASTRUCTURE ONLY.

A numpy restatement of the reference's algorithm for the HiMuon optimizer
step (tang0389/himuon, src/himuon/optimizers/himuon.py and
src/himuon/triton_kernels/*). Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py may import it, and only as the checker or the
reported CPU baseline; the product path (himuon_amd) never does.

Functions and the reference lines they restate:

  bf16_round            torch's float32 -> bfloat16 cast (round to nearest even)
  momentum              himuon.py:350-357 (_compute_momentum)
  tile / untile         himuon.py:288-310 (_tile/_untile), 704-719 (gather into
                        the concat buffer), 315-329 (_post_ns_per_param)
  tile_source_map       closed-form index map of tile/untile (himuon.py:704-719)
  balanced_chunks       himuon.py:459-481
  auto_b_hw             himuon.py:376-403
  plan_buckets          himuon.py:483-586
  ns5_fp64              the quintic NS without rounding (muon.py:14-44,
                        test_kernels.py:176-198 with exact arithmetic)
  ns5_spectral          the same map through an SVD (closed form used to pin
                        ns5_fp64)
  xxt / ba_plus_caa / bmm_add / ns_iteration
                        the three products of one NS iteration at the
                        reference kernels' rounding points (XXT.py:55-75,
                        ba_plus_cAA.py:58-85, fused_bmm_add.py:73-88; the
                        2-D third product torch.addmm, himuon.py:249-253)
  ns5_staged            NS with the rounding points of the HIP kernels and the
                        reference kernels: bf16 after every GEMM stage, fp32
                        accumulation (ns5_smem.py:84-101, XXT.py:62-70,
                        ba_plus_cAA.py:78-85, fused_bmm_add.py:73-88)
  ns5_staged_2d         ns5_staged with the 2-D third product of
                        himuon.py:249-253 (torch.addmm: bf16(B X + a X),
                        one rounding)
  ns5_eager             NS with the rounding of the eager-torch oracle of
                        tests/integration/test_kernels.py:176-198 (every torch
                        op rounds to bf16)
  lr_scale              himuon.py:181-186
  fma32 / round_to      correctly rounded fp32 fma; cast to a param dtype
  apply_update_eager    the reference's eager WD/LR form (himuon.py:342-348)
  apply_update          WD/LR of himuon.py:215-228 / 333-348 as torch's GPU
                        kernels evaluate p.mul_(1-lr*wd) then p.add_(u,
                        alpha=-lr): u rounded to the param dtype, then one
                        fp32 fma, then rounded
  lerp32 / adamw_bias / adamw_step
                        AdamW fallback step, himuon.py:359-372 (torch's lerp
                        as an fma; every op rounded to the moment dtype)
  step_param            one optimizer step on a list of params
                        (himuon.py:978-1046, 333-348; graph-mode scaling of
                        himuon.py:337-341 / 222-228)

Pinning (tests/test_oracle.py): bf16_round against torch's cast; momentum
against torch's in-place ops; tile maps against brute-force loops and
committed integer tables; chunks against their invariants and the survey's
worked values; ns5_fp64 against its SVD closed form, rank-1 and diagonal
closed forms, orthogonal invariance and transpose symmetry; ns5_staged and
ns5_eager against ns5_fp64 (bf16-sized distance) and the singular-value band;
fma32 against exact rational arithmetic; apply_update against torch's CPU ops
for fp32 params (bit-exact) and, in tests/test_gpu_apply.py, against torch's
GPU ops for bf16 and fp32 params (each element equals torch's bulk form or its
remainder form) and for fp16 params over torch's vectorised bulk path
(bit-exact; torch's non-vectorised tail rounds a few fp16 elements by neither
form). lerp32 against torch's CPU lerp (both weight branches,
bit-exact); adamw_step against torch's CPU ops: bf16 moments and update and
fp32 moments bit-exact (torch's CPU fp32 sqrt is not correctly rounded, so
the fp32 update is pinned within 2 ulp there), adamw_bias against its
float64 closed form; on the GPU (tests/test_gpu_adamw.py) the kernel's
moments and update equal adamw_step given the kernel's bias corrections, and
the kernel equals torch's GPU ops bit for bit.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

NS_A, NS_B, NS_C = 3.4445, -4.7750, 2.0315  # himuon.py:237, ns5_smem.py:26-28
NS_EPS = 1e-7  # himuon.py:242, ns5_smem.py:30

F32 = np.float32


# ---------------------------------------------------------------------------
# Rounding
# ---------------------------------------------------------------------------
def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned
    as float32. NaN -> canonical quiet NaN."""
    x = np.ascontiguousarray(np.asarray(x, dtype=F32))
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, 0x7FC0, r).astype(np.uint32) << 16
    return r.view(F32).reshape(x.shape)


def f16_round(x) -> np.ndarray:
    return np.asarray(x, dtype=F32).astype(np.float16).astype(F32)


def fma32(a, b, c) -> np.ndarray:
    """Correctly rounded float32 fused multiply-add a*b + c.

    a*b is exact in float64 (24+24 bits); the float64 sum is made exact with
    TwoSum and rounded to odd, after which one rounding to float32 is correct
    (53 >= 24 + 2)."""
    a, b, c = (np.asarray(v, dtype=F32).astype(np.float64) for v in (a, b, c))
    p = a * b
    s = p + c
    bb = s - p
    e = (p - (s - bb)) + (c - bb)  # exact error: p + c = s + e
    inexact = e != 0
    even = (s.view(np.uint64) & 1) == 0
    bump = inexact & even & np.isfinite(s)
    s = np.where(bump, np.nextafter(s, np.where(e > 0, np.inf, -np.inf)), s)
    return s.astype(F32)


def round_to(x, dtype: str) -> np.ndarray:
    if dtype == "float32":
        return np.asarray(x, dtype=F32)
    if dtype == "bfloat16":
        return bf16_round(x)
    if dtype == "float16":
        return f16_round(x)
    raise ValueError(dtype)


# ---------------------------------------------------------------------------
# Momentum (himuon.py:350-357)
# ---------------------------------------------------------------------------
def momentum(g, buf, mu: float, nesterov: bool, dtype: str = "float32"):
    """buf <- buf*mu + g (two in-place ops, each stored in ``dtype``);
    g_eff = g + mu*buf (one op: torch's add with alpha, a fused multiply-add
    in fp32, stored once) if nesterov else buf. Returns (g_eff, new_buf)."""
    g = np.asarray(g, dtype=F32)
    buf = np.asarray(buf, dtype=F32)
    m = F32(mu)
    nb = round_to(round_to(buf * m, dtype) + g, dtype)
    if nesterov:
        ge = round_to(fma32(m, nb, g), dtype)
    else:
        ge = nb
    return ge, nb


# ---------------------------------------------------------------------------
# Tiling (himuon.py:288-310, 704-719, 315-329)
# ---------------------------------------------------------------------------
def tile_grid(h: int, w: int, tile_h: int, tile_w: int) -> tuple[int, int]:
    """(R, C) = padded shape // tile (himuon.py:546-551)."""
    pad_h = (tile_h - h % tile_h) % tile_h
    pad_w = (tile_w - w % tile_w) % tile_w
    return (h + pad_h) // tile_h, (w + pad_w) // tile_w


def tile(x: np.ndarray, tile_h: int, tile_w: int) -> np.ndarray:
    """(h, w) -> (R*C, tile_h, tile_w), zero padded bottom/right; tile (r, c)
    at index r*C + c holds x[r*Th:(r+1)*Th, c*Tw:(c+1)*Tw]."""
    h, w = x.shape
    R, C = tile_grid(h, w, tile_h, tile_w)
    pad = np.zeros((R * tile_h, C * tile_w), dtype=x.dtype)
    pad[:h, :w] = x
    return pad.reshape(R, tile_h, C, tile_w).transpose(0, 2, 1, 3).reshape(R * C, tile_h, tile_w)


def untile(tiles: np.ndarray, h: int, w: int) -> np.ndarray:
    """Inverse of ``tile``: (R*C, Th, Tw) -> (h, w)."""
    _, tile_h, tile_w = tiles.shape
    R, C = tile_grid(h, w, tile_h, tile_w)
    full = tiles.reshape(R, C, tile_h, tile_w).transpose(0, 2, 1, 3).reshape(R * tile_h, C * tile_w)
    return full[:h, :w]


def tile_source_map(h: int, w: int, tile_h: int, tile_w: int) -> np.ndarray:
    """Integer table src[t, i, j] = row*w + col of the parameter element at
    tile t position (i, j), or -1 for padding."""
    R, C = tile_grid(h, w, tile_h, tile_w)
    t = np.arange(R * C)
    r, c = t // C, t % C
    i = np.arange(tile_h)
    j = np.arange(tile_w)
    row = r[:, None, None] * tile_h + i[None, :, None]
    col = c[:, None, None] * tile_w + j[None, None, :]
    ok = (row < h) & (col < w)
    return np.where(ok, row * w + col, -1).astype(np.int64)


def ns_operand(tile_hw: np.ndarray) -> np.ndarray:
    """NS operand of a (..., Th, Tw) tile: its transpose when tall
    (himuon.py:240-241, 276-278)."""
    return np.swapaxes(tile_hw, -1, -2) if tile_hw.shape[-2] > tile_hw.shape[-1] else tile_hw


# ---------------------------------------------------------------------------
# Plan (himuon.py:376-403, 459-586)
# ---------------------------------------------------------------------------
def balanced_chunks(B_total: int, b_hw: int) -> list[int]:
    if B_total <= 0:
        return []
    n = -(-B_total // b_hw)
    out, rem = [], B_total
    for i in range(n):
        c = -(-rem // (n - i))
        out.append(c)
        rem -= c
    return out


def auto_b_hw(T: int, dtype_bytes: int, total_mem: int | None, override: int | None = None,
              fraction: float = 0.15) -> int:
    if total_mem is None:  # no device: himuon.py:390-393
        return max(1, int(override)) if override is not None else 1
    cap = max(1, int(fraction * total_mem) // (4 * T * T * dtype_bytes))
    return max(1, min(int(override), cap)) if override is not None else cap


@dataclass
class PlanParam:
    shape: tuple[int, int]
    tile: tuple[int, int]
    dtype_bytes: int = 4
    dtype: str = "float32"


def plan_buckets(params: list[PlanParam], total_mem: int | None, override: int | None = None) -> list[dict]:
    """Buckets keyed (Th, Tw, dtype) in parameter order; full-NS params
    (numel <= Th*Tw) are skipped (himuon.py:541-544)."""
    by_key: dict[tuple, list[int]] = {}
    counts: dict[int, int] = {}
    for idx, p in enumerate(params):
        h, w = p.shape
        th, tw = p.tile
        if h * w <= th * tw:
            continue
        R, C = tile_grid(h, w, th, tw)
        counts[idx] = R * C
        by_key.setdefault((th, tw, p.dtype), []).append(idx)
    plan = []
    for (th, tw, dt), idxs in by_key.items():
        B_total = sum(counts[i] for i in idxs)
        b_hw = auto_b_hw(max(th, tw), params[idxs[0]].dtype_bytes, total_mem, override)
        chunks = balanced_chunks(B_total, b_hw)
        plan.append({"key": (th, tw, dt), "params": idxs, "tile_counts": [counts[i] for i in idxs],
                     "B_total": B_total, "B_hw": b_hw, "chunk_sizes": chunks, "n_calls": len(chunks)})
    return plan


# ---------------------------------------------------------------------------
# Newton-Schulz
# ---------------------------------------------------------------------------
def quintic(s, steps: int = 5, coeffs=(NS_A, NS_B, NS_C)):
    """The scalar map sigma -> a s + b s^3 + c s^5 applied ``steps`` times."""
    a, b, c = coeffs
    s = np.asarray(s, dtype=np.float64)
    for _ in range(steps):
        s = a * s + b * s**3 + c * s**5
    return s


def quintic_band(smin: float, smax: float = 1.0, steps: int = 5, coeffs=(NS_A, NS_B, NS_C)):
    """(lo, hi) of the iterated quintic over normalised sigma in [smin, smax]:
    the band every output singular value of a tile lies in when its
    normalised input spectrum lies in [smin, smax]."""
    smin = max(float(smin), 1e-12)
    s = np.concatenate([np.geomspace(smin, smax, 200001), [smin, smax]])
    f = quintic(s, steps, coeffs)
    return float(f.min()), float(f.max())


def ns5_fp64(G, steps: int = 5, coeffs=(NS_A, NS_B, NS_C), eps: float = NS_EPS) -> np.ndarray:
    """Quintic NS in float64 without rounding; (..., M, N) -> same shape."""
    a, b, c = coeffs
    X = np.asarray(G, dtype=np.float64)
    tall = X.shape[-2] > X.shape[-1]
    if tall:
        X = np.swapaxes(X, -1, -2)
    X = X / (np.sqrt((X * X).sum(axis=(-2, -1), keepdims=True)) + eps)
    for _ in range(steps):
        A = X @ np.swapaxes(X, -1, -2)
        B = b * A + c * (A @ A)
        X = a * X + B @ X
    if tall:
        X = np.swapaxes(X, -1, -2)
    return X


def ns5_spectral(G, steps: int = 5, coeffs=(NS_A, NS_B, NS_C), eps: float = NS_EPS) -> np.ndarray:
    """Closed form of ns5_fp64 via the SVD G = U S V^T:
    NS(G) = U quintic(S / (||G||_F + eps)) V^T."""
    G = np.asarray(G, dtype=np.float64)
    U, S, Vt = np.linalg.svd(G, full_matrices=False)
    nrm = np.sqrt((G * G).sum(axis=(-2, -1), keepdims=True))[..., 0]
    f = quintic(S / (nrm + eps), steps, coeffs)
    return (U * f[..., None, :]) @ Vt


def _mm32(x: np.ndarray, y: np.ndarray) -> np.ndarray:
    """float32 product with float32 accumulation (bf16 inputs are exact in fp32)."""
    return np.matmul(x.astype(F32), y.astype(F32))


def xxt(X) -> np.ndarray:
    """A = bf16(X X^T), fp32 accumulation (XXT.py:55-75)."""
    return bf16_round(_mm32(X, np.swapaxes(X, -1, -2)))


def ba_plus_caa(A, alpha: float, beta: float) -> np.ndarray:
    """B = bf16(alpha * (A A^T) + beta * A), fp32 accumulation and epilogue
    (ba_plus_cAA.py:58-85)."""
    return bf16_round(F32(alpha) * _mm32(A, np.swapaxes(A, -1, -2)) + F32(beta) * np.asarray(A, F32))


def bmm_add(B, X, a: float, round_once: bool = False) -> np.ndarray:
    """X' = bf16(bf16(B X) + a X) (fused_bmm_add.py:73-88, the batched form),
    or with round_once bf16(B X + a X) from the fp32 product, one rounding
    (torch.addmm(X, B, X, beta=a), the 2-D form of himuon.py:249-253)."""
    X = np.asarray(X, F32)
    if round_once:
        return bf16_round(fma32(F32(a), X, _mm32(B, X)))
    return bf16_round(bf16_round(_mm32(B, X)) + F32(a) * X)


def ns_iteration(X, coeffs=(NS_A, NS_B, NS_C), round_once: bool = False):
    """One NS iteration at the kernels' rounding points: (A, B, X')."""
    a, b, c = coeffs
    A = xxt(X)
    B = ba_plus_caa(A, c, b)
    return A, B, bmm_add(B, X, a, round_once)


def ns5_staged(G, steps: int = 5, coeffs=(NS_A, NS_B, NS_C), eps: float = NS_EPS,
               round_once: bool = False) -> np.ndarray:
    """NS with the kernel rounding points; (..., M, N) float32 -> float32
    holding bf16 values.

        X0 = bf16(x * (1 / (||x||_F + eps)))     x = bf16(G), norm in fp32
        A  = bf16(X X^T)
        B  = bf16(c * (A A^T) + b * A)
        X  = bf16(bf16(B X) + a * X)             batched (3-D) form, fused_bmm_add
        X  = bf16(B X + a * X)                   round_once: the 2-D form,
                                                 torch.addmm(X, B, X, beta=a)
                                                 (himuon.py:249-253)
    """
    a, b, c = (F32(v) for v in coeffs)
    X = bf16_round(np.asarray(G, dtype=F32))
    tall = X.shape[-2] > X.shape[-1]
    if tall:
        X = np.ascontiguousarray(np.swapaxes(X, -1, -2))
    nrm = np.sqrt((X.astype(F32) ** 2).sum(axis=(-2, -1), keepdims=True, dtype=F32)).astype(F32)
    inv = (F32(1.0) / (nrm + F32(eps))).astype(F32)
    X = bf16_round(X * inv)
    for _ in range(steps):
        _, _, X = ns_iteration(X, coeffs, round_once)
    if tall:
        X = np.ascontiguousarray(np.swapaxes(X, -1, -2))
    return X


def ns5_staged_2d(G, steps: int = 5, coeffs=(NS_A, NS_B, NS_C), eps: float = NS_EPS) -> np.ndarray:
    """ns5_staged with the reference's 2-D third product (one rounding of
    B X + a X, torch.addmm; himuon.py:249-253): what newton_schulz computes
    for a 2-D input and the full-matrix path (himuon.py:861) for each
    parameter. Batched inputs are treated as independent 2-D matrices."""
    return ns5_staged(G, steps, coeffs, eps, round_once=True)


def ns5_eager(G, steps: int = 5, coeffs=(NS_A, NS_B, NS_C), eps: float = NS_EPS) -> np.ndarray:
    """NS with the rounding of the eager torch oracle (test_kernels.py:176-198):
    every torch op on bf16 tensors rounds its result to bf16."""
    a, b, c = (F32(v) for v in coeffs)
    X = bf16_round(np.asarray(G, dtype=F32))
    tall = X.shape[-2] > X.shape[-1]
    if tall:
        X = np.ascontiguousarray(np.swapaxes(X, -1, -2))
    nrm = bf16_round(np.sqrt((X**2).sum(axis=(-2, -1), keepdims=True, dtype=F32)))
    den = bf16_round(nrm + F32(eps))
    X = bf16_round(X / den)
    for _ in range(steps):
        A = bf16_round(_mm32(X, np.swapaxes(X, -1, -2)))
        B = bf16_round(bf16_round(b * A) + bf16_round(c * bf16_round(_mm32(A, A))))
        X = bf16_round(bf16_round(a * X) + bf16_round(_mm32(B, X)))
    if tall:
        X = np.ascontiguousarray(np.swapaxes(X, -1, -2))
    return X


# ---------------------------------------------------------------------------
# Update (himuon.py:181-186, 333-348, 215-228)
# ---------------------------------------------------------------------------
def lr_scale(block_shape, lr_adjust: str = "tile") -> float:
    if lr_adjust == "none":
        return 1.0
    return 0.2 * math.sqrt(max(block_shape[0], block_shape[1]))


def apply_update(p, update, lr: float, wd: float, dtype: str = "float32",
                 update_dtype: str = "float32") -> np.ndarray:
    """p.mul_(1 - lr*wd) (if wd > 0), then p.add_(update, alpha=-lr), each
    stored in the parameter dtype (himuon.py:222-228, 345-348). torch's
    in-place add computes in the parameter's dtype: the update is first
    rounded to it, then `p + alpha * u` is one fp32 fused multiply-add. For
    fp16 parameters with an fp32 update (the optimizer's fp32 grads) torch's
    mixed-dtype add rounds that multiply-add once from the exact value
    instead of through fp32 (measured on the GPU over 1 M elements); numpy's
    float64 -> float16 conversion is that single rounding, and the float64
    value is exact (a 35-bit product plus an fp16 term)."""
    p = np.asarray(p, dtype=F32)
    if wd > 0.0:
        p = round_to(p * F32(1 - lr * wd), dtype)
    u = round_to(np.asarray(update, dtype=F32), dtype)
    if dtype == "float16" and update_dtype == "float32":
        exact = np.float64(F32(-lr)) * u.astype(np.float64) + p.astype(np.float64)
        return exact.astype(np.float16).astype(F32)
    return round_to(fma32(F32(-lr), u, p), dtype)


def apply_update_eager(p, ns_out, lr: float, wd: float, scale: float, dtype: str = "float32") -> np.ndarray:
    """The reference's eager WD/LR form (himuon.py:342-348): the update is the
    unscaled NS output and the lr-adjust scale rides in the alpha,
    p.mul_(1 - lr*wd); p.add_(u, alpha=-lr*scale) (alpha formed in double,
    then fp32). This build always applies the graph form (update scaled
    first, alpha = -lr: apply_update), which for bf16 parameters rounds the
    scaled update to bf16 before the add, as the reference's graph path does;
    the two differ by at most that rounding (2^-8 of lr |u s|) plus one unit
    in the last place (bound pinned in tests/test_oracle.py)."""
    p = np.asarray(p, dtype=F32)
    if wd > 0.0:
        p = round_to(p * F32(1 - lr * wd), dtype)
    u = round_to(np.asarray(ns_out, dtype=F32), dtype)
    return round_to(fma32(F32(-lr * scale), u, p), dtype)


# ---------------------------------------------------------------------------
# AdamW fallback (himuon.py:359-372, 878-888)
# ---------------------------------------------------------------------------
def lerp32(a, b, w) -> np.ndarray:
    """torch's lerp with a scalar weight in fp32 opmath: fma(w, b - a, a) for
    |w| < 0.5, else fma(-(b - a), 1 - w, b) (the form torch's kernels take;
    ATen Lerp.h, is_lerp_weight_small)."""
    a = np.asarray(a, dtype=F32)
    b = np.asarray(b, dtype=F32)
    w = F32(w)
    d = (b - a).astype(F32)
    if abs(float(w)) < 0.5:
        return fma32(w, d, a)
    return fma32(-d, F32(1) - w, b)


def adamw_bias(beta: float, step) -> F32:
    """1 - beta ** step in fp32 with a correctly rounded pow (step is the
    fp32 counter after its increment). The reference evaluates the power with
    the device math library's powf, which is not correctly rounded: it may
    differ from this in the last bit at some steps."""
    pw = F32(np.float64(F32(beta)) ** np.float64(F32(step)))
    return F32(F32(1) - pw)


def adamw_step(g, m, v, step, betas, eps, dtype: str = "float32", bias=None):
    """One AdamW fallback step (himuon.py:359-372) as torch's GPU kernels
    evaluate it, every op's result stored in the moment dtype (= grad dtype):

        step += 1
        m = lerp(m, g, 1 - b1); v = lerp(v, g*g, 1 - b2)
        update = (m / bc1) / (sqrt(v) / sqrt(bc2) + eps)

    1 - beta is formed in double (a Python float) and then rounded to fp32, as
    the lerp weight is. bc1 and sqrt(bc2) are fp32 0-dim tensors there, which
    the GPU kernels cast to the moment dtype before dividing (a CPU scalar
    operand would keep fp32); the Python-float eps enters in fp32. ``bias`` =
    (bc1, sqrt(bc2)) overrides the bias corrections (for a comparison that
    takes them from the device). Returns (update, m, v, step, (bc1,
    sqrt(bc2))) with the fp32 bias corrections."""
    b1, b2 = betas
    s = F32(F32(step) + F32(1))
    g = round_to(np.asarray(g, dtype=F32), dtype)
    m = round_to(lerp32(m, g, F32(1.0 - b1)), dtype)
    v = round_to(lerp32(v, round_to(g * g, dtype), F32(1.0 - b2)), dtype)
    if bias is None:
        bc1 = adamw_bias(b1, s)
        sbc2 = np.sqrt(adamw_bias(b2, s), dtype=F32)
    else:
        bc1, sbc2 = F32(bias[0]), F32(bias[1])
    t1 = round_to(m / round_to(bc1, dtype), dtype)
    t2 = round_to(np.sqrt(v, dtype=F32), dtype)
    t3 = round_to(round_to(t2 / round_to(sbc2, dtype), dtype) + F32(eps), dtype)
    # (fp16: eps = 1e-8 underflows, so t3 is 0 where v is; x / 0 gives the IEEE inf/NaN torch gives)
    with np.errstate(divide="ignore", invalid="ignore"):
        u = round_to(t1 / t3, dtype)
    return u, m, v, s, (bc1, sbc2)


@dataclass
class OracleParam:
    p: np.ndarray            # float32 values of the parameter
    g: np.ndarray            # float32 values of the gradient
    buf: np.ndarray | None   # momentum buffer (None -> zeros)
    tile: tuple[int, int]
    lr: float = 0.02
    wd: float = 0.1
    mu: float = 0.95
    nesterov: bool = True
    ns_steps: int = 5
    p_dtype: str = "float32"
    g_dtype: str = "float32"
    lr_adjust: str = "tile"


def step_param(op: OracleParam, ns=ns5_staged):
    """One HiMuon step of one parameter. Returns (new_p, new_buf, update)."""
    buf = np.zeros_like(op.g) if op.buf is None else op.buf
    ge, nb = momentum(op.g, buf, op.mu, op.nesterov, op.g_dtype)
    h, w = ge.shape
    th, tw = op.tile
    if h * w <= th * tw:  # full-NS path (himuon.py:852-874): a 2-D NS call
        u = ns(ge, op.ns_steps, round_once=True) if ns is ns5_staged else ns(ge, op.ns_steps)
        scale = lr_scale((h, w), op.lr_adjust)
    else:
        tiles = tile(ge, th, tw)
        u = untile(ns(tiles, op.ns_steps), h, w)
        scale = lr_scale((th, tw), op.lr_adjust)
    # update tensor in grad dtype, scaled in-graph (himuon.py:257, 338-341)
    upd = round_to(round_to(u, op.g_dtype) * F32(scale), op.g_dtype)
    newp = apply_update(op.p, upd, op.lr, op.wd, op.p_dtype, op.g_dtype)
    return newp, nb, upd
