"""NS5 with the untile and WD/LR fused into its last iteration
(himuon_ns5_untile_apply) against the two launches it replaces
(himuon_ns5_ex, then himuon_untile_apply; himuon.py:232-284, 315-348) on the
same inputs: parameters bit-identical.

Two copies of one bucket of 512 x 512 NS tiles: ragged right and bottom
edges (partial tiles), a parameter narrower than a tile, an unaligned row
stride (a column slice, so some 8-element vectors take the element-wise
path), two param groups with their own (1 - lr wd, -lr) and lr scales. The
fused side runs in two chunks (tile_begin != 0) with sub-batches smaller than
a chunk, so the tile numbering of the untile is offset inside each launch.
fp32 and bf16 parameters, fp32 and bf16 grads, step counts 2 and 5, both
rounding forms of the third product.
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
SHAPES = [(1024, 1536), (700, 900), (512, 2048), (600, 1000), (512, 512)]


def _groups_table():
    sa = torch.zeros(2 * nat.APPLY_MAX_GROUPS, device=DEV, dtype=torch.float32)
    nat.write_scale_alpha(sa, [1.0 - LR * WD, 1.0 - 0.5 * LR * 0.3], [-LR, -0.5 * LR])
    return sa


def _pair(shapes, gdt, pdt, round_once, seed):
    """Two identical fused tile groups over their own copies of the data."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    params = [(torch.randn(h, w, device=DEV, generator=g) * 0.02).to(pdt) for h, w in shapes]
    grads = [(torch.randn(h, w, device=DEV, generator=g) * 1e-3).to(gdt) for h, w in shapes]
    moms = [(torch.randn(h, w, device=DEV, generator=g) * 1e-3).to(gdt) for h, w in shapes]
    out = []
    for _ in range(2):
        ps = [p.clone() for p in params]
        if len(shapes) > 3:  # one parameter with an unaligned row stride (a column slice)
            h, w = shapes[3]
            wide = torch.zeros(h, w + 3, device=DEV, dtype=pdt)
            wide[:, :w] = params[3]
            ps[3] = wide[:, :w]
        grp = TileGroup(ps, [q.clone() for q in grads], [m.clone() for m in moms], 512, 512,
                        upd_scales=[float(O.lr_scale(s)) for s in shapes], mus=[0.95] * len(ps),
                        nesterovs=[True] * len(ps), device=torch.device(DEV), dtype=gdt,
                        apply_groups=[i % 2 for i in range(len(ps))], round_once=round_once)
        out.append((ps, grp))
    return out, params


@pytest.mark.parametrize("gdt,pdt", [(F32, BF16), (F32, F32), (BF16, BF16)], ids=["f32-bf16", "f32-f32", "bf16-bf16"])
@pytest.mark.parametrize("steps", [2, 5])
@pytest.mark.parametrize("round_once", [False, True], ids=["batched", "2d"])
def test_ns_untile_equals_ns_then_untile(gdt, pdt, steps, round_once):
    print(f"[ns untile] {gdt} {pdt} steps={steps} round_once={round_once}", flush=True)
    ((p_sep, g_sep), (p_fus, g_fus)), p0s = _pair(SHAPES, gdt, pdt, round_once, seed=steps + 7 * round_once)
    assert g_fus.ns_untile_ok(steps) and not g_fus.ns_untile_ok(1)
    sa = _groups_table()
    n = g_sep.n_tiles
    sb = 5  # sub-batches smaller than a chunk: the untile's tile numbering is offset per launch
    ws = torch.empty(nat.ns5_workspace_bytes(sb, 512, 512), device=DEV, dtype=torch.uint8)
    g_sep.gather()
    g_sep.ns(0, n, steps, ws, sb)
    g_sep.untile(steps, sa)
    g_fus.gather()
    k = 11
    g_fus.ns_untile(0, k, steps, ws, sb, sa)
    g_fus.ns_untile(k, n - k, steps, ws, sb, sa)
    torch.cuda.synchronize()
    for i, (a, b, p0) in enumerate(zip(p_sep, p_fus, p0s)):
        nd = int((a != b).sum())
        assert nd == 0, f"param {i} {tuple(a.shape)}: {nd} elements differ"
        assert bool((b != p0).any()), f"param {i} was not updated"


@pytest.mark.parametrize("gdt,pdt", [(F32, BF16), (F32, F32)], ids=["f32-bf16", "f32-f32"])
def test_ns_untile_many_edge_tiles(gdt, pdt):
    """Enough tiles that every workgroup runs several work items, most of them
    on tiles with ragged edges: items whose 32-row blocks go element by
    element (some issuing no memory operation at all) are followed by further
    items whose A panel was loaded during their epilogue."""
    print(f"[ns untile, many edge tiles] {gdt} {pdt}", flush=True)
    shapes = [(700, 900), (1000, 600), (520, 1030), (600, 1000)] * 16
    ((p_sep, g_sep), (p_fus, g_fus)), p0s = _pair(shapes, gdt, pdt, False, seed=11)
    assert g_fus.n_tiles >= 256
    sa = _groups_table()
    n = g_sep.n_tiles
    ws = torch.empty(nat.ns5_workspace_bytes(n, 512, 512), device=DEV, dtype=torch.uint8)
    g_sep.gather()
    g_sep.ns(0, n, 5, ws, n)
    g_sep.untile(5, sa)
    g_fus.gather()
    g_fus.ns_untile(0, n, 5, ws, n, sa)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(p_sep, p_fus)):
        nd = int((a != b).sum())
        assert nd == 0, f"param {i} {tuple(a.shape)}: {nd} elements differ"


def test_ns_untile_falls_back_where_it_does_not_apply():
    """Geometries the fused path does not take are refused before any launch
    (the optimizer then runs NS and the untile as two launches)."""
    ((_, g), _), _ = _pair([(512, 512)], F32, BF16, False, 3)
    sa = _groups_table()
    ws = torch.empty(nat.ns5_workspace_bytes(1, 512, 512), device=DEV, dtype=torch.uint8)
    with pytest.raises(RuntimeError):
        nat.ns5_untile_apply(g.tiles, g.alt, g.inv, 1, 512, 512, 1, ws, 1, g.desc, 1, 0, 512, 512, BF16, sa)
    with pytest.raises(RuntimeError):
        nat.ns5_untile_apply(g.tiles, g.alt, g.inv, 1, 512, 512, 5, ws, 1, g.desc, 1, 0, 512, 512, BF16, sa,
                             family="stream3")
    assert not nat.ns5_untile_apply_supported(512, 512, 512, 512, 5, torch.float16)
    assert not nat.ns5_untile_apply_supported(256, 512, 256, 512, 5, BF16)
