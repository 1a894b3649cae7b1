"""ctypes binding of libhimuon_hip.so (the C ABI declared in include/himuon_hip.h).

Host-side plumbing only: pointers come from ``tensor.data_ptr()``, launches go
to ``torch.cuda.current_stream()`` so they are recorded by ``torch.cuda.graph``
capture. The library is required: every entry point raises ``RuntimeError`` if
it is missing or the call fails (the reference raises the same way when its
GPU kernels are unavailable, src/himuon/triton_kernels/__init__.py:8-19).
"""

from __future__ import annotations

import ctypes
import math
from ctypes import c_float, c_int, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libhimuon_hip.so"

ABI_VERSION = 5
NS_ALIGN = 128
DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
# Operand dtypes of the typed stage products (himuon_*_typed): the above and fp8 e5m2.
PRODUCT_IN_CODES = {**DTYPE_CODES, **({torch.float8_e5m2: 3} if hasattr(torch, "float8_e5m2") else {})}

# Quintic coefficients and normaliser epsilon (himuon.py:237,242; ns5_smem.py:26-30).
NS_A, NS_B, NS_C = 3.4445, -4.7750, 2.0315
NS_EPS = 1e-7


class ParamDesc(ctypes.Structure):
    """Mirror of HimuonParamDesc (include/himuon_hip.h)."""

    _fields_ = [
        ("grad", c_void_p),
        ("momentum", c_void_p),
        ("update", c_void_p),
        ("h", c_int64),
        ("w", c_int64),
        ("ld_grad", c_int64),
        ("ld_mom", c_int64),
        ("ld_upd", c_int64),
        ("tile0", c_int64),
        ("R", c_int32),
        ("C", c_int32),
        ("upd_scale", c_float),
        ("mu", c_float),
        ("nesterov", c_int32),
        ("group", c_int32),
    ]


assert ctypes.sizeof(ParamDesc) == 96


class ApplyDesc(ctypes.Structure):
    """Mirror of HimuonApplyDesc (include/himuon_hip.h)."""

    _fields_ = [
        ("param", c_void_p),
        ("update", c_void_p),
        ("numel", c_int64),
        ("chunk0", c_int64),
        ("group", c_int32),
        ("reserved", c_int32),
    ]


assert ctypes.sizeof(ApplyDesc) == 40
APPLY_MAX_GROUPS = 32


class AdamwDesc(ctypes.Structure):
    """Mirror of HimuonAdamwDesc (include/himuon_hip.h)."""

    _fields_ = [
        ("grad", c_void_p),
        ("moment1", c_void_p),
        ("moment2", c_void_p),
        ("update", c_void_p),
        ("step", c_void_p),
        ("numel", c_int64),
        ("chunk0", c_int64),
        ("group", c_int32),
        ("reserved", c_int32),
    ]


assert ctypes.sizeof(AdamwDesc) == 64
ADAMW_MAX_GROUPS = 32

# name -> (restype, argtypes)
_SIGNATURES = {
    "himuon_abi_version": (c_int, []),
    "himuon_error_string": (ctypes.c_char_p, [c_int]),
    "himuon_gather_partials_per_tile": (c_int, [c_int, c_int, c_int, c_int]),
    "himuon_momentum_gather": (
        c_int,
        [c_void_p, c_int, c_int64, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p],
    ),
    "himuon_tile_scale": (c_int, [c_void_p, c_int, c_int64, c_float, c_void_p, c_void_p]),
    "himuon_ns5_workspace_bytes": (c_size_t, [c_int64, c_int, c_int]),
    "himuon_ns5": (
        c_int,
        [
            c_void_p,
            c_void_p,
            c_void_p,
            c_int64,
            c_int,
            c_int,
            c_int,
            c_float,
            c_float,
            c_float,
            c_void_p,
            c_size_t,
            c_int64,
            c_void_p,
        ],
    ),
    "himuon_ns5_ex": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_float, c_float, c_float, c_void_p,
         c_size_t, c_int64, c_int, c_void_p],
    ),
    "himuon_xxt": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_void_p]),
    "himuon_ba_plus_caa": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_float, c_float, c_int, c_void_p]),
    "himuon_bmm_add": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_float, c_int, c_void_p]),
    "himuon_ba_bmm_add": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_float, c_float, c_float,
                                  c_int, c_void_p]),
    "himuon_xxt_typed": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p]),
    "himuon_ba_plus_caa_typed": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_float, c_float, c_int, c_int,
                                         c_void_p]),
    "himuon_bmm_add_typed": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_float, c_int, c_int,
                                     c_void_p]),
    "himuon_lds_step": (c_int, [c_void_p, c_int, c_int64, c_int64, c_int, c_int, c_int, c_int, c_int, c_float,
                                c_float, c_float, c_float, c_int, c_void_p, c_void_p]),
    "himuon_ns5_noalloc": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_float, c_float,
                                   c_float, c_int, c_void_p]),
    "himuon_untile": (
        c_int,
        [c_void_p, c_int, c_int64, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p],
    ),
    "himuon_ns5_untile_apply_supported": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_int]),
    "himuon_ns5_untile_apply": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_float, c_float, c_float, c_void_p,
         c_size_t, c_int64, c_int, c_void_p, c_int, c_int64, c_int, c_int, c_int, c_void_p, c_void_p],
    ),
    "himuon_untile_apply": (
        c_int,
        [c_void_p, c_int, c_int64, c_int, c_int, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p],
    ),
    "himuon_write_scale_alpha": (
        c_int, [c_void_p, ctypes.POINTER(c_float), ctypes.POINTER(c_float), c_int, c_void_p],
    ),
    "himuon_apply_chunk_elems": (c_int64, []),
    "himuon_apply_updates": (
        c_int,
        [c_void_p, c_int, c_int64, c_int, c_int, ctypes.POINTER(c_float), ctypes.POINTER(c_float), c_int,
         c_void_p],
    ),
    "himuon_adamw_chunk_elems": (c_int64, []),
    "himuon_adamw_step": (
        c_int,
        [c_void_p, c_int, c_int64, c_int, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double),
         ctypes.POINTER(ctypes.c_double), c_int, c_void_p, c_void_p],
    ),
}

_lib = None


def lib_path() -> Path:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load the library once; raise RuntimeError if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    path = lib_path()
    if not path.exists():
        raise RuntimeError(
            f"libhimuon_hip.so not found at {path}. Build it with `python -m himuon_amd.build` "
            "(hipcc --offload-arch=gfx950). HiMuon has no CPU fallback."
        )
    lib = ctypes.CDLL(str(path))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.himuon_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"libhimuon_hip.so ABI {ver} != expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().himuon_error_string(rc).decode()
        raise RuntimeError(f"{what} failed: {msg} (code {rc})")


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"HiMuon HIP path supports float32/bfloat16/float16 grads, got {dtype}")


# ---------------------------------------------------------------------------
# Geometry
# ---------------------------------------------------------------------------
def round_up(x: int, a: int) -> int:
    return (x + a - 1) // a * a


def ns_geometry(tile_h: int, tile_w: int) -> tuple[int, int, int, int, bool]:
    """(m, n, mp, np, transposed) of the NS operand for a tile_h x tile_w tile:
    NS runs on the tile's transpose when it is tall (himuon.py:240-241,276-278)."""
    trans = tile_h > tile_w
    m, n = (tile_w, tile_h) if trans else (tile_h, tile_w)
    return m, n, round_up(m, NS_ALIGN), round_up(n, NS_ALIGN), trans


def gather_partials_per_tile(tile_h: int, tile_w: int, mp: int, np_: int) -> int:
    n = load().himuon_gather_partials_per_tile(tile_h, tile_w, mp, np_)
    _check(0 if n > 0 else n, "himuon_gather_partials_per_tile")
    return n


def ns5_workspace_bytes(sub_batch: int, mp: int, np_: int) -> int:
    return int(load().himuon_ns5_workspace_bytes(sub_batch, mp, np_))


# himuon_ns5_ex flags (include/himuon_hip.h). Kernel families: AUTO picks per
# geometry (what the optimizer runs); BLOCK128 runs the 128x128-block kernels
# everywhere and STREAM3 the three streamed products where AUTO fuses two
# (comparison runs, named explicitly by the caller). ROUND_ONCE: the
# reference's 2-D third product, bf16(B X + a X).
NS_FAMILY_AUTO = 0
NS_FAMILY_BLOCK128 = 1
NS_FAMILY_STREAM3 = 2
NS_ROUND_ONCE = 0x10
NS_FAMILIES = {"auto": NS_FAMILY_AUTO, "block128": NS_FAMILY_BLOCK128, "stream3": NS_FAMILY_STREAM3}
# HIMUON_NS_ROWS(m): the NS operands' real row count, when at most 64 (small-M
# tiles iterate at their own height instead of the padded mp = 128).
NS_ROWS_SHIFT = 8
NS_ROWS_MAX = 64


def few_rows_supported(m: int, mp: int, np_: int) -> bool:
    """Whether family AUTO runs m-row NS operands at their own height (the
    dispatch rule of himuon_ns5_ex with HIMUON_NS_ROWS(m)): mp == 128, np a
    multiple of 128 (of 256 above 512) up to 2048 (m <= 16) or 1024
    (16 < m <= 32); 32 < m <= 64 at np = 128 only."""
    if mp != 128 or not 0 < m <= NS_ROWS_MAX:
        return False
    if m > 32:
        return np_ == 128
    if np_ in (128, 256, 384, 512):
        return True
    if m <= 32 and np_ in (768, 1024):
        return True
    return m <= 16 and np_ in (1536, 2048)


def default_sub_batch(n_tiles: int, mp: int, np_: int) -> int:
    """Tiles per NS sub-batch (one set of launches): about 2 GiB of bf16 NS
    operand (4096 tiles of 512x512), so each launch has >10k 256x256 blocks
    and launch tails stay small; the A/B workspace is twice that."""
    target = 2 << 30
    return max(1, min(n_tiles, target // (mp * np_ * 2)))


# ---------------------------------------------------------------------------
# Descriptor tables
# ---------------------------------------------------------------------------
def make_desc_table(descs: list[ParamDesc], device) -> torch.Tensor:
    """Copy an array of ParamDesc to device memory (uint8 tensor)."""
    arr = (ParamDesc * len(descs))(*descs)
    host = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
    return host.to(device)


# ---------------------------------------------------------------------------
# Entry points
# ---------------------------------------------------------------------------
def momentum_gather(desc_table, n_params, n_tiles, tile_h, tile_w, mp, np_, dtype, tiles, partials):
    _check(
        load().himuon_momentum_gather(
            desc_table.data_ptr(),
            n_params,
            n_tiles,
            tile_h,
            tile_w,
            mp,
            np_,
            dtype_code(dtype),
            tiles.data_ptr(),
            partials.data_ptr(),
            _stream(),
        ),
        "himuon_momentum_gather",
    )


def tile_scale(partials, per_tile, n_tiles, inv, eps=NS_EPS):
    _check(
        load().himuon_tile_scale(partials.data_ptr(), per_tile, n_tiles, eps, inv.data_ptr(), _stream()),
        "himuon_tile_scale",
    )


def ns5(x, y, inv, n_tiles, mp, np_, steps, workspace, sub_batch, coeffs=(NS_A, NS_B, NS_C), family="auto",
        round_once=False, rows=0):
    """NS5 on tiles x; X ping-pongs into y: the result is in x for an even
    step count and in y for an odd one. ``family``: a key of NS_FAMILIES;
    ``round_once`` selects the 2-D rounding of the third product; ``rows``: the
    NS operands' real row count (0: unknown or above NS_ROWS_MAX)."""
    a, b, c = coeffs
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    flags = _ns_flags(family, round_once, rows)
    _check(
        load().himuon_ns5_ex(
            x.data_ptr(), y.data_ptr(), inv.data_ptr(), n_tiles, mp, np_, steps, a, b, c,
            ws_ptr, ws_bytes, sub_batch, flags, _stream(),
        ),
        "himuon_ns5",
    )


def _ns_flags(family, round_once, rows) -> int:
    flags = _stage_flags(family, round_once)
    if 0 < rows <= NS_ROWS_MAX:
        flags |= rows << NS_ROWS_SHIFT
    return flags


def ns5_untile_apply_supported(mp, np_, tile_h, tile_w, steps, param_dtype, family="auto", round_once=False):
    """True when himuon_ns5_untile_apply takes this geometry (512 x 512 NS
    tiles, not transposed, family AUTO, steps >= 2, fp32 or bf16 parameters)."""
    if param_dtype not in DTYPE_CODES:
        return False
    return bool(load().himuon_ns5_untile_apply_supported(mp, np_, tile_h, tile_w, steps,
                                                         _stage_flags(family, round_once),
                                                         DTYPE_CODES[param_dtype]))


def ns5_untile_apply(x, y, inv, n_tiles, mp, np_, steps, workspace, sub_batch, desc_table, n_params, tile_begin,
                     tile_h, tile_w, param_dtype, scale_alpha, coeffs=(NS_A, NS_B, NS_C), family="auto",
                     round_once=False, rows=0):
    """NS5 of bucket tiles tile_begin .. tile_begin + n_tiles - 1 (x, y: the
    tile buffers advanced to tile_begin) with the untile with the WD/LR of
    scale_alpha fused into the last iteration: the parameters the descriptors
    point at are updated in place; x and y hold no NS result afterwards."""
    a, b, c = coeffs
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    _check(
        load().himuon_ns5_untile_apply(
            x.data_ptr(), y.data_ptr(), inv.data_ptr(), n_tiles, mp, np_, steps, a, b, c, ws_ptr, ws_bytes,
            sub_batch, _ns_flags(family, round_once, rows), desc_table.data_ptr(), n_params, tile_begin, tile_h,
            tile_w, dtype_code(param_dtype), scale_alpha.data_ptr(), _stream(),
        ),
        "himuon_ns5_untile_apply",
    )


def _stage_flags(family="auto", round_once=False) -> int:
    return NS_FAMILIES[family] | (NS_ROUND_ONCE if round_once else 0)


def xxt(x, out, batch, M, K, family="auto"):
    _check(load().himuon_xxt(x.data_ptr(), out.data_ptr(), batch, M, K, _stage_flags(family), _stream()),
           "himuon_xxt")


def ba_plus_caa(a, out, batch, M, alpha, beta, family="auto"):
    _check(load().himuon_ba_plus_caa(a.data_ptr(), out.data_ptr(), batch, M, alpha, beta, _stage_flags(family),
                                     _stream()), "himuon_ba_plus_caa")


def bmm_add(b, x, out, batch, M, N, a, round_once=False, family="auto"):
    _check(load().himuon_bmm_add(b.data_ptr(), x.data_ptr(), out.data_ptr(), batch, M, N, a,
                                 _stage_flags(family, round_once), _stream()), "himuon_bmm_add")


def xxt_typed(x, out, batch, M, K):
    """out = x x^T for any operand dtype of PRODUCT_IN_CODES, out fp32/bf16/fp16."""
    _check(load().himuon_xxt_typed(x.data_ptr(), out.data_ptr(), batch, M, K, PRODUCT_IN_CODES[x.dtype],
                                   DTYPE_CODES[out.dtype], _stream()), "himuon_xxt_typed")


def ba_plus_caa_typed(a, out, batch, M, alpha, beta):
    """out = alpha a a^T + beta a, any operand dtype of PRODUCT_IN_CODES."""
    _check(load().himuon_ba_plus_caa_typed(a.data_ptr(), out.data_ptr(), batch, M, alpha, beta,
                                           PRODUCT_IN_CODES[a.dtype], DTYPE_CODES[out.dtype], _stream()),
           "himuon_ba_plus_caa_typed")


def bmm_add_typed(b, x, out, batch, M, N, a):
    """out = out_dtype(b x) + a x, any operand dtype of PRODUCT_IN_CODES."""
    if b.dtype != x.dtype:
        raise TypeError(f"bmm_add_typed: operands of one dtype expected, got {b.dtype} and {x.dtype}")
    _check(load().himuon_bmm_add_typed(b.data_ptr(), x.data_ptr(), out.data_ptr(), batch, M, N, a,
                                       PRODUCT_IN_CODES[x.dtype], DTYPE_CODES[out.dtype], _stream()),
           "himuon_bmm_add_typed")


def ba_bmm_add(a, x, out, batch, alpha, beta, gamma, round_once=False):
    """out = bf16(bf16(B X) + gamma X), B = bf16(alpha A A^T + beta A) kept on
    chip (512 x 512 tiles; bf16(B X + gamma X) with round_once)."""
    _check(load().himuon_ba_bmm_add(a.data_ptr(), x.data_ptr(), out.data_ptr(), batch, 512, 512, alpha, beta, gamma,
                                    NS_ROUND_ONCE if round_once else 0, _stream()), "himuon_ba_bmm_add")


def lds_step_supported(tile_h: int, tile_w: int, dtype, param_dtype) -> bool:
    """Buckets himuon_lds_step takes: 128 x 128 NS tiles without transpose,
    fp32/bf16 grads and parameters."""
    return (0 < tile_h <= tile_w <= 128 and dtype in (torch.float32, torch.bfloat16)
            and param_dtype in (torch.float32, torch.bfloat16))


def lds_step(desc_table, n_params, tile_begin, n_tiles, tile_h, tile_w, dtype, param_dtype, steps, scale_alpha,
             round_once=False, coeffs=(NS_A, NS_B, NS_C), eps=NS_EPS):
    """Momentum, gather, normaliser, NS5 and the untile with WD/LR for bucket
    tiles tile_begin .. + n_tiles - 1 in one launch (128 x 128 NS tiles)."""
    a, b, c = coeffs
    _check(
        load().himuon_lds_step(
            desc_table.data_ptr(), n_params, tile_begin, n_tiles, tile_h, tile_w, dtype_code(dtype),
            dtype_code(param_dtype), steps, a, b, c, eps, NS_ROUND_ONCE if round_once else 0,
            scale_alpha.data_ptr(), _stream(),
        ),
        "himuon_lds_step",
    )


def untile(desc_table, n_params, n_tiles, tile_h, tile_w, mp, np_, dtype, tiles):
    _check(
        load().himuon_untile(
            desc_table.data_ptr(),
            n_params,
            n_tiles,
            tile_h,
            tile_w,
            mp,
            np_,
            dtype_code(dtype),
            tiles.data_ptr(),
            _stream(),
        ),
        "himuon_untile",
    )


def untile_apply(desc_table, n_params, n_tiles, tile_h, tile_w, mp, np_, param_dtype, tiles, scale_alpha):
    """Untile with the group's WD/LR applied in place to the parameters the
    descriptors point at; scale_alpha: fp32 device tensor (s_g, alpha_g) per
    group, read when the kernel runs."""
    _check(
        load().himuon_untile_apply(
            desc_table.data_ptr(), n_params, n_tiles, tile_h, tile_w, mp, np_, dtype_code(param_dtype),
            tiles.data_ptr(), scale_alpha.data_ptr(), _stream(),
        ),
        "himuon_untile_apply",
    )


def write_scale_alpha(table, scales, alphas):
    """(s_g, alpha_g) per group into the fp32 device table the fused untile
    reads, as a kernel on the current stream (no host synchronisation)."""
    n = len(scales)
    if n != len(alphas) or not 0 < n <= APPLY_MAX_GROUPS or table.numel() < 2 * n:
        raise ValueError(f"write_scale_alpha: {n} groups for a table of {table.numel()} floats")
    if table.dtype != torch.float32 or not table.is_cuda:
        raise TypeError("write_scale_alpha: table must be an fp32 device tensor")
    cs = (c_float * n)(*scales)
    ca = (c_float * n)(*alphas)
    _check(load().himuon_write_scale_alpha(table.data_ptr(), cs, ca, n, _stream()), "himuon_write_scale_alpha")


def lr_scale(block_shape, lr_adjust: str = "tile") -> float:
    """adjust_lr_for_muon(1.0, block) (himuon.py:181-186)."""
    if lr_adjust == "none":
        return 1.0
    a, b = block_shape[:2]
    return 0.2 * math.sqrt(max(a, b))


def apply_updates(desc_table, n_descs, n_chunks, param_dtype, update_dtype, scales, alphas):
    """One launch of the WD + LR application over a descriptor table
    (himuon.py:215-228); scales/alphas are per-group host floats."""
    n = len(scales)
    s_arr = (c_float * n)(*scales)
    a_arr = (c_float * n)(*alphas)
    _check(
        load().himuon_apply_updates(
            desc_table.data_ptr(), n_descs, n_chunks, DTYPE_CODES[param_dtype], DTYPE_CODES[update_dtype],
            s_arr, a_arr, n, _stream(),
        ),
        "himuon_apply_updates",
    )


def apply_desc_table(descs: list[ApplyDesc], device) -> torch.Tensor:
    arr = (ApplyDesc * len(descs))(*descs)
    host = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
    return host.to(device)


def adamw_chunk_elems() -> int:
    return int(load().himuon_adamw_chunk_elems())


def adamw_step(desc_table, n_descs, n_chunks, dtype, beta1s, beta2s, epss, bias):
    """One AdamW fallback step over a descriptor table (himuon.py:359-372):
    per-group betas/eps are host Python floats; ``bias`` is fp32 device
    scratch of 2 * n_descs elements."""
    n = len(beta1s)
    b1 = (ctypes.c_double * n)(*beta1s)
    b2 = (ctypes.c_double * n)(*beta2s)
    ep = (ctypes.c_double * n)(*epss)
    _check(
        load().himuon_adamw_step(
            desc_table.data_ptr(), n_descs, n_chunks, DTYPE_CODES[dtype], b1, b2, ep, n, bias.data_ptr(), _stream()
        ),
        "himuon_adamw_step",
    )


def adamw_desc_table(descs: list[AdamwDesc], device) -> torch.Tensor:
    arr = (AdamwDesc * len(descs))(*descs)
    host = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8)
    return host.to(device)
