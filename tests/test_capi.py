"""CPU checks of the C ABI: libhimuon_hip.so loads, exports every function
include/himuon_hip.h declares, agrees on the descriptor layout, and rejects bad
arguments on the host before launching anything (no GPU needed)."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from himuon_amd import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "himuon_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(himuon_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not nat.lib_path().exists():
        pytest.fail(f"{nat.lib_path()} missing: run `python -m himuon_amd.build`")
    return nat.load()


def test_exports_every_declared_symbol(lib):
    declared = _declared_functions()
    assert declared, "no functions parsed from the header"
    out = subprocess.run(["nm", "-D", "--defined-only", str(nat.lib_path())], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (himuon_\w+)", out))
    assert set(declared) <= exported, set(declared) - exported
    assert set(declared) == set(nat.exported_symbols())
    for name in declared:
        assert hasattr(lib, name)


def test_abi_version_and_errors(lib):
    assert lib.himuon_abi_version() == nat.ABI_VERSION
    assert lib.himuon_error_string(0) == b"success"
    assert b"invalid" in lib.himuon_error_string(-22)
    assert b"workspace" in lib.himuon_error_string(-28)


def test_desc_layout_matches_header():
    # offsets of HimuonParamDesc fields (include/himuon_hip.h)
    d = nat.ParamDesc
    assert ctypes.sizeof(d) == 96
    assert d.tile0.offset == 64 and d.R.offset == 72 and d.upd_scale.offset == 80
    assert d.mu.offset == 84 and d.nesterov.offset == 88


def test_adamw_desc_layout_matches_header():
    # offsets of HimuonAdamwDesc fields (include/himuon_hip.h)
    d = nat.AdamwDesc
    assert ctypes.sizeof(d) == 64
    assert d.update.offset == 24 and d.step.offset == 32 and d.numel.offset == 40
    assert d.chunk0.offset == 48 and d.group.offset == 56
    a = nat.ApplyDesc
    assert ctypes.sizeof(a) == 40 and a.chunk0.offset == 24 and a.group.offset == 32


def test_adamw_argument_errors(lib):
    z = None
    one = (ctypes.c_double * 1)(0.95)
    many = (ctypes.c_double * 40)(*([0.95] * 40))
    assert lib.himuon_adamw_chunk_elems() > 0
    # null descriptor table or bias scratch
    assert lib.himuon_adamw_step(z, 1, 4, 0, one, one, one, 1, 8, z) == -22
    assert lib.himuon_adamw_step(8, 1, 4, 0, one, one, one, 1, z, z) == -22
    # unknown dtype code, too many groups, missing host arrays
    assert lib.himuon_adamw_step(8, 1, 4, 9, one, one, one, 1, 8, z) == -22
    assert lib.himuon_adamw_step(8, 1, 4, 0, many, many, many, 40, 8, z) == -22
    assert lib.himuon_adamw_step(8, 1, 4, 0, z, one, one, 1, 8, z) == -22


def test_scale_alpha_argument_errors(lib):
    z = None
    one = (ctypes.c_float * 1)(1.0)
    many = (ctypes.c_float * 40)(*([1.0] * 40))
    # null table or host arrays, no groups, more groups than the table holds
    assert lib.himuon_write_scale_alpha(z, one, one, 1, z) == -22
    assert lib.himuon_write_scale_alpha(8, z, one, 1, z) == -22
    assert lib.himuon_write_scale_alpha(8, one, z, 1, z) == -22
    assert lib.himuon_write_scale_alpha(8, one, one, 0, z) == -22
    assert lib.himuon_write_scale_alpha(8, many, many, 33, z) == -22
    # the fused untile needs its (scale, alpha) table
    assert lib.himuon_untile_apply(8, 1, 4, 512, 512, 512, 512, 1, 8, z, z) == -22


def test_partials_per_tile(lib):
    assert lib.himuon_gather_partials_per_tile(512, 512, 512, 512) == 512 // 32  # 32-row slabs
    assert lib.himuon_gather_partials_per_tile(256, 1024, 256, 1024) == 256 // 32
    assert lib.himuon_gather_partials_per_tile(128, 128, 128, 128) == 1  # whole 128x128 tiles
    assert lib.himuon_gather_partials_per_tile(256, 256, 256, 256) == 4  # 64-row slabs
    assert lib.himuon_gather_partials_per_tile(1024, 512, 512, 1024) == (512 // 64) * (1024 // 64)  # tall: 64x64 blocks
    assert lib.himuon_gather_partials_per_tile(512, 512, 500, 512) == -22  # not aligned
    assert lib.himuon_gather_partials_per_tile(512, 512, 384, 512) == -22  # mp < m
    # np = 384: 32-row slabs (16384 / 384 = 42 rows would not divide mp = 128)
    assert lib.himuon_gather_partials_per_tile(100, 300, 128, 384) == 4


def test_plain_slabs_cover_every_padded_row(lib):
    # Plain-tile gather work items are slabs of mp / P rows; they must tile the
    # whole padded height (padding rows are written as zero by the gather), so
    # the row count divides mp for every NS geometry, and a slab holds at most
    # 16384 elements unless 32 rows already exceed that.
    for mp in range(128, 2049, 128):
        for np_ in range(mp, 4097, 128):
            p = lib.himuon_gather_partials_per_tile(mp, np_, mp, np_)
            assert p > 0 and mp % p == 0, (mp, np_, p)
            rows = mp // p
            assert rows in (32, 64, 128) and rows <= mp, (mp, np_, rows)
            assert rows * np_ <= 16384 or rows == 32, (mp, np_, rows)


def test_workspace_bytes(lib):
    assert lib.himuon_ns5_workspace_bytes(4, 512, 512) == 2 * 4 * 512 * 512 * 2  # A and B
    assert lib.himuon_ns5_workspace_bytes(0, 512, 512) == 0


def test_argument_errors_return_before_launch(lib):
    z = None
    # null descriptor / buffers
    assert lib.himuon_momentum_gather(z, 1, 4, 512, 512, 512, 512, 0, z, z, z) == -22
    # bad dtype code with otherwise valid (dummy) pointers: still rejected on the host
    assert lib.himuon_momentum_gather(8, 1, 4, 512, 512, 512, 512, 9, 8, 8, z) == -22
    # mp > np is not an NS geometry
    assert lib.himuon_ns5(8, 16, 8, 4, 1024, 512, 5, 1.0, 1.0, 1.0, 8, 1 << 30, 4, z) == -22
    # x and y must be distinct
    assert lib.himuon_ns5(8, 8, 8, 4, 512, 512, 5, 1.0, 1.0, 1.0, 8, 1 << 30, 4, z) == -22
    # workspace too small
    assert lib.himuon_ns5(8, 16, 8, 4, 512, 512, 5, 1.0, 1.0, 1.0, 8, 16, 4, z) == -28
    assert lib.himuon_untile(z, 1, 4, 512, 512, 512, 512, 0, z, z) == -22
    assert lib.himuon_tile_scale(z, 16, 4, 1e-7, z, z) == -22
    # empty work is a no-op success
    assert lib.himuon_tile_scale(8, 16, 0, 1e-7, 8, z) == 0


def test_ns5_ex_and_stage_argument_errors(lib):
    z = None
    # unknown flag bits or family codes
    assert lib.himuon_ns5_ex(8, 16, 8, 4, 512, 512, 5, 1.0, 1.0, 1.0, 8, 1 << 30, 4, 0x40, z) == -22
    assert lib.himuon_ns5_ex(8, 16, 8, 4, 512, 512, 5, 1.0, 1.0, 1.0, 8, 1 << 30, 4, 7, z) == -22
    # the flags that exist are accepted (empty work returns before any launch)
    assert lib.himuon_ns5_ex(8, 16, 8, 0, 512, 512, 5, 1.0, 1.0, 1.0, 8, 1 << 30, 4, 0x11, z) == 0
    # stage products: null pointers, unaligned dimensions, aliasing, bad flags
    assert lib.himuon_xxt(z, 8, 1, 256, 256, 0, z) == -22
    assert lib.himuon_xxt(8, 16, 1, 200, 256, 0, z) == -22
    assert lib.himuon_xxt(8, 16, 1, 256, 256, 0x10, z) == -22  # round-once is for bmm_add only
    assert lib.himuon_ba_plus_caa(8, 8, 1, 256, 1.0, 1.0, 0, z) == -22
    assert lib.himuon_ba_plus_caa(8, 16, 1, 100, 1.0, 1.0, 0, z) == -22
    assert lib.himuon_bmm_add(8, 16, 16, 1, 256, 256, 1.0, 0, z) == -22
    assert lib.himuon_bmm_add(8, 16, 24, 1, 256, 200, 1.0, 0, z) == -22
    assert lib.himuon_bmm_add(8, 16, 24, 1, 256, 256, 1.0, 0x20, z) == -22
    assert lib.himuon_bmm_add(8, 16, 24, 0, 256, 256, 1.0, 0x10, z) == 0
    # the fused second and third products: 512 x 512 only, no aliasing, round-once only
    assert lib.himuon_ba_bmm_add(8, 16, 24, 1, 256, 256, 1.0, 1.0, 1.0, 0, z) == -22
    assert lib.himuon_ba_bmm_add(8, 16, 24, 1, 512, 1024, 1.0, 1.0, 1.0, 0, z) == -22
    assert lib.himuon_ba_bmm_add(8, 16, 16, 1, 512, 512, 1.0, 1.0, 1.0, 0, z) == -22
    assert lib.himuon_ba_bmm_add(8, 16, 24, 1, 512, 512, 1.0, 1.0, 1.0, 1, z) == -22
    # 32-bit work-item indices (4 per tile): 2^29 - 1 tiles at most
    assert lib.himuon_ba_bmm_add(8, 16, 24, (1 << 29) + 1, 512, 512, 1.0, 1.0, 1.0, 0, z) == -22
    assert lib.himuon_ba_bmm_add(8, 16, 24, 1 << 29, 512, 512, 1.0, 1.0, 1.0, 0, z) == -22
    assert lib.himuon_ba_bmm_add(8, 16, 24, 0, 512, 512, 1.0, 1.0, 1.0, 0x10, z) == 0
    # the typed stage products: operand dtypes 0..3 (fp8 e5m2 = 3), output 0..2,
    # M (and N) multiples of 128, K of 64, no aliasing, at most 2^31 - 8 blocks
    assert lib.himuon_xxt_typed(8, 16, 0, 128, 64, 3, 2, z) == 0  # empty batch: no launch
    assert lib.himuon_xxt_typed(8, 16, 1, 128, 64, 4, 2, z) == -22
    assert lib.himuon_xxt_typed(8, 16, 1, 128, 64, 3, 3, z) == -22  # no fp8 output
    assert lib.himuon_xxt_typed(8, 16, 1, 100, 64, 0, 0, z) == -22
    assert lib.himuon_xxt_typed(8, 16, 1, 128, 96, 0, 0, z) == -22
    assert lib.himuon_xxt_typed(8, 8, 1, 128, 64, 0, 0, z) == -22
    assert lib.himuon_xxt_typed(8, 16, 1 << 31, 128, 64, 0, 0, z) == -22
    assert lib.himuon_ba_plus_caa_typed(8, 16, 1, 200, 1.0, 1.0, 2, 2, z) == -22
    assert lib.himuon_ba_plus_caa_typed(0, 16, 1, 128, 1.0, 1.0, 2, 2, z) == -22
    assert lib.himuon_bmm_add_typed(8, 16, 16, 1, 128, 128, 1.0, 2, 2, z) == -22
    assert lib.himuon_bmm_add_typed(8, 16, 24, 1, 128, 100, 1.0, 2, 2, z) == -22
    assert lib.himuon_bmm_add_typed(8, 16, 24, 1, 128, 128, 1.0, 2, -1, z) == -22
    assert lib.himuon_bmm_add_typed(8, 16, 24, 1 << 31, 128, 128, 1.0, 2, 2, z) == -22
    assert lib.himuon_bmm_add_typed(8, 16, 24, 0, 128, 128, 1.0, 3, 0, z) == 0
    # the LDS-resident step: tile_h <= tile_w <= 128, fp32/bf16 grads and parameters,
    # a descriptor table and a (scale, alpha) table, round-once the only flag
    def lds(prm=8, npar=1, base=0, n=0, th=128, tw=128, dt=0, pdt=1, steps=5, flags=0x10, sa=16):
        return lib.himuon_lds_step(prm, npar, base, n, th, tw, dt, pdt, steps, 1.0, 1.0, 1.0, 1e-7, flags, sa, z)
    assert lds() == 0 and lds(th=64, tw=100, dt=1, pdt=0, steps=0) == 0  # empty work: no launch
    for bad in (dict(th=256), dict(tw=256), dict(th=100, tw=64), dict(dt=2), dict(pdt=2), dict(steps=-1),
                dict(flags=1), dict(prm=z), dict(npar=0), dict(sa=z), dict(base=-1), dict(n=-1), dict(th=0)):
        assert lds(**bad) == -22, bad
    # NS with the untile fused into its last iteration: 512 x 512 NS tiles, not
    # transposed, family AUTO (the 2-D rounding allowed), steps >= 2, fp32/bf16
    # parameters, a descriptor table and a (scale, alpha) table
    sup = lib.himuon_ns5_untile_apply_supported
    assert sup(512, 512, 512, 512, 5, 0, 1) and sup(512, 512, 300, 500, 2, 0x10, 0)
    for args in ((256, 512, 256, 512, 5, 0, 1), (512, 1024, 512, 1024, 5, 0, 1), (512, 512, 500, 300, 5, 0, 1),
                 (512, 512, 512, 512, 1, 0, 1), (512, 512, 512, 512, 5, 1, 1), (512, 512, 512, 512, 5, 2, 1),
                 (512, 512, 512, 512, 5, 0, 2), (512, 512, 600, 600, 5, 0, 1), (512, 512, 0, 512, 5, 0, 1)):
        assert not sup(*args), args

    def nsu(n=0, mp=512, np_=512, steps=5, flags=0, prm=8, npar=2, base=0, th=512, tw=512, pdt=1, sa=16):
        return lib.himuon_ns5_untile_apply(8, 16, 24, n, mp, np_, steps, 1.0, 1.0, 1.0, 32, 1 << 30, 4, flags, prm,
                                           npar, base, th, tw, pdt, sa, z)
    assert nsu() == 0 and nsu(flags=0x10, th=400, pdt=0) == 0  # empty work: no launch
    for bad in (dict(mp=256), dict(steps=1), dict(flags=1), dict(th=513), dict(pdt=2), dict(prm=z), dict(npar=0),
                dict(base=-1), dict(sa=z), dict(th=512, tw=500)):
        assert nsu(**bad) == -22, bad


def test_geometry_helpers():
    assert nat.ns_geometry(512, 512) == (512, 512, 512, 512, False)
    assert nat.ns_geometry(768, 513) == (513, 768, 640, 768, True)
    assert nat.ns_geometry(64, 64) == (64, 64, 128, 128, False)
    assert nat.ns_geometry(1024, 3072) == (1024, 3072, 1024, 3072, False)
