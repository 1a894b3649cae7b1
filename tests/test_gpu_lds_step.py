"""The whole step of a 128 x 128-tile bucket in one launch (himuon_lds_step)
against the four launches it replaces (himuon_momentum_gather,
himuon_tile_scale, himuon_ns5_ex, himuon_untile_apply; himuon.py:704-719,
232-284, 315-348) on the same inputs: momentum buffers and parameters
bit-identical.

Two copies of one bucket: ragged right and bottom edges, a parameter smaller
than one tile, an unaligned row stride, two param groups with their own
(1 - lr wd, -lr). The fused side runs in two chunks (tile_begin != 0). Every
dtype pair the entry point takes, Nesterov on and off, no momentum buffer,
step counts 0 to 5, both rounding forms of the third product, and a
whole-matrix group (tile = the matrix, h <= w <= 128).
"""

from __future__ import annotations

import pytest
import torch

from oracle import himuon_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from himuon_amd import _native as nat
    from himuon_amd.engine import TileGroup

DEV = "cuda"
F32, BF16 = torch.float32, torch.bfloat16
LR, WD = 0.02, 0.1


def _groups_table():
    sa = torch.zeros(2 * nat.APPLY_MAX_GROUPS, device=DEV, dtype=torch.float32)
    nat.write_scale_alpha(sa, [1.0 - LR * WD, 1.0 - 0.5 * LR * 0.3], [-LR, -0.5 * LR])
    return sa


def _pair(shapes, th, tw, gdt, pdt, nesterov, with_mom, round_once, seed):
    """Two identical fused tile groups over their own copies of the data."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    params = [(torch.randn(h, w, device=DEV, generator=g) * 0.02).to(pdt) for h, w in shapes]
    grads = [(torch.randn(h, w, device=DEV, generator=g) * 1e-3).to(gdt) for h, w in shapes]
    moms = [(torch.randn(h, w, device=DEV, generator=g) * 1e-3).to(gdt) for h, w in shapes]
    out = []
    for _ in range(2):
        ps = [p.clone() for p in params]
        if len(shapes) > 2:  # one parameter with an unaligned row stride (a column slice)
            h, w = shapes[2]
            wide = torch.zeros(h, w + 3, device=DEV, dtype=pdt)
            wide[:, :w] = params[2]
            ps[2] = wide[:, :w]
        ms = [m.clone() for m in moms] if with_mom else [None] * len(shapes)
        grp = TileGroup(ps, [q.clone() for q in grads], ms, th, tw,
                        upd_scales=[float(O.lr_scale((th, tw)))] * len(ps), mus=[0.9] * len(ps),
                        nesterovs=[nesterov] * len(ps), device=torch.device(DEV), dtype=gdt,
                        apply_groups=[i % 2 for i in range(len(ps))], round_once=round_once)
        out.append((ps, ms, grp))
    return out


def _run_and_compare(shapes, th, tw, gdt, pdt, nesterov=True, with_mom=True, round_once=False, steps=5,
                     split=5, seed=0):
    (p_sep, m_sep, g_sep), (p_fus, m_fus, g_fus) = _pair(shapes, th, tw, gdt, pdt, nesterov, with_mom,
                                                          round_once, seed)
    assert g_fus.lds_step_ok()
    sa = _groups_table()
    n = g_sep.n_tiles
    sb = max(1, n // 3)
    ws = torch.empty(max(1, nat.ns5_workspace_bytes(sb, g_sep.mp, g_sep.np)), device=DEV, dtype=torch.uint8)
    g_sep.gather()
    g_sep.ns(0, n, steps, ws, sb)
    g_sep.untile(steps, sa)
    k = min(split, n)
    g_fus.lds_step(0, k, steps, sa)
    g_fus.lds_step(k, n - k, steps, sa)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(p_sep, p_fus)):
        nd = int((a != b).sum())
        assert nd == 0, f"param {i} {tuple(a.shape)}: {nd} elements differ"
        assert bool((b != 0).any())
    if with_mom:
        for i, (a, b) in enumerate(zip(m_sep, m_fus)):
            assert torch.equal(a, b), f"momentum {i} differs"


SHAPES = [(300, 200), (128, 128), (256, 390), (77, 130)]


@pytest.mark.parametrize("gdt,pdt", [(F32, F32), (F32, BF16), (BF16, BF16), (BF16, F32)],
                         ids=["f32-f32", "f32-bf16", "bf16-bf16", "bf16-f32"])
@pytest.mark.parametrize("steps", [0, 1, 2, 5])
def test_lds_step_equals_the_four_launches(gdt, pdt, steps):
    print(f"[lds step] {gdt} {pdt} steps={steps}", flush=True)
    _run_and_compare(SHAPES, 128, 128, gdt, pdt, steps=steps, seed=steps)


@pytest.mark.parametrize("nesterov,with_mom", [(False, True), (True, False)], ids=["plain-momentum", "no-momentum"])
def test_lds_step_momentum_forms(nesterov, with_mom):
    _run_and_compare(SHAPES, 128, 128, F32, BF16, nesterov=nesterov, with_mom=with_mom, seed=11)


def test_lds_step_round_once_and_rectangular_tiles():
    # tile 64 x 128 (wide, no transpose): NS operand 64 x 128 in a 128 x 128 tile
    _run_and_compare([(200, 300), (64, 128), (130, 260)], 64, 128, F32, F32, round_once=True, seed=12)


def test_lds_step_whole_matrix_group():
    # the full-matrix form: each matrix one tile (tile = the matrix), 2-D rounding
    _run_and_compare([(100, 120)], 100, 120, F32, BF16, round_once=True, split=0, seed=13)


def test_lds_step_refuses_other_buckets():
    sa = _groups_table()
    (_, _, g), _ = _pair([(256, 256)], 128, 128, F32, F32, True, True, False, 1)
    lib = nat.load()
    z = None
    args = (g.desc.data_ptr(), 1, 0, 4, 128, 128, 0, 0, 5, 1.0, 1.0, 1.0, 1e-7, 0, sa.data_ptr(), z)
    assert lib.himuon_lds_step(*args) == 0
    for pos, val in [(4, 256), (5, 256), (4, 100), (6, 2), (7, 2), (8, -1), (13, 1), (2, -1)]:
        a = list(args)
        a[pos] = val
        if pos == 4 and val == 100:
            a[5] = 64  # tile_h > tile_w: a transposed tile
        assert lib.himuon_lds_step(*a) == -22, (pos, val)
    torch.cuda.synchronize()
