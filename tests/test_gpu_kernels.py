"""GPU parity of the HIP kernels against the CPU oracle and torch references.

* gather (momentum + tile + bf16 cast): bit-exact momentum buffers and NS tiles
  against oracle.momentum / oracle.tile, every padding and transpose case;
* untile: bit-exact updates against oracle.untile times the lr scale;
* NS5: per-tile relative Frobenius error against the reference's NS5 in the
  same dtypes (torch on the GPU) and against the CPU oracle, plus the
  singular-value band of every tile.

Inputs are generated on the CPU from fixed seeds and copied to the device.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import himuon_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from himuon_amd import _native as nat
    from himuon_amd.engine import TileGroup, newton_schulz

    from gpu_ref import ns5_torch_eager, ns5_torch_staged, per_tile_rel_fro, well_conditioned

DEV = "cuda"
TDT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def _cpu_randn(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def _ns_layout(tiles_hw: np.ndarray, mp: int, np_: int) -> np.ndarray:
    """(n, Th, Tw) tiles -> (n, mp, np) NS operands (transposed if tall, zero padded)."""
    n, th, tw = tiles_hw.shape
    x = np.swapaxes(tiles_hw, 1, 2) if th > tw else tiles_hw
    out = np.zeros((n, mp, np_), dtype=np.float32)
    out[:, : x.shape[1], : x.shape[2]] = x
    return out


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    if t.dtype == torch.float32:
        return t.numpy().view(np.uint32)
    return t.view(torch.int16).numpy().view(np.uint16)


GATHER_CASES = [
    # (name, [param shapes], tile_h, tile_w, dtype, nesterov)
    ("square_256_fp32", [(1024, 1024)], 256, 256, "float32", True),
    ("pad_512_fp32", [(768, 513), (513, 768)], 512, 512, "float32", True),
    ("tall_tiles_fp32", [(300, 200), (128, 64)], 128, 64, "float32", True),
    ("wide_tiles_bf16", [(200, 300)], 64, 128, "bfloat16", True),
    ("multi_bf16_plain", [(512, 1024), (256, 512), (1024, 2048)], 256, 256, "bfloat16", False),
    ("fp16", [(384, 640)], 128, 128, "float16", True),
    ("full_tall_fp32", [(2048, 1024)], 2048, 1024, "float32", True),
    ("odd_small", [(7, 50), (50, 7)], 16, 16, "float32", True),
    ("nt_512_mixed", [(1024, 1536), (700, 300)], 512, 512, "float32", True),
    ("nt_tall_tiles", [(1024, 512)], 512, 256, "bfloat16", True),
    # np = 384 (padded rows 100..127 are written by the last 32-row slab)
    ("full_wide_384", [(100, 300)], 100, 300, "float32", True),
    ("wide_384_bf16", [(256, 700)], 128, 300, "bfloat16", True),
]


@pytest.fixture(params=["auto", "stream3", "block128"])
def ns_family(request):
    """Run a test under each NS kernel family selection, passed explicitly
    to newton_schulz / TileGroup: "auto" (the product's per-geometry choice:
    LDS-resident, the fused GramB/Apply kernel for 512 x 512 tiles, persistent
    streamed 256-blocks or 128-blocks), "stream3" (the three streamed products
    where AUTO fuses two) and "block128" (the 128-block kernels for every
    geometry)."""
    return request.param


def _make_group(shapes, th, tw, dtype, nesterov, seed, mus=None, with_mom=True):
    tdt = TDT[dtype]
    grads = [_cpu_randn(s, seed + i, 1e-3, tdt).to(DEV) for i, s in enumerate(shapes)]
    moms = [_cpu_randn(s, seed + 100 + i, 1e-3, tdt).to(DEV) if with_mom else None for i, s in enumerate(shapes)]
    mus = mus or [0.95] * len(shapes)
    grp = TileGroup(
        params=grads, grads=grads, moms=moms, tile_h=th, tile_w=tw,
        upd_scales=[O.lr_scale((th, tw))] * len(shapes), mus=mus,
        nesterovs=[nesterov] * len(shapes), device=torch.device(DEV), dtype=tdt,
    )
    return grp, grads, moms


@pytest.mark.parametrize("name,shapes,th,tw,dtype,nesterov", GATHER_CASES, ids=[c[0] for c in GATHER_CASES])
def test_gather_bit_exact(name, shapes, th, tw, dtype, nesterov):
    print(f"[gather] {name}", flush=True)
    mus = [0.95, 0.9, 0.8][: len(shapes)]
    grp, grads, moms = _make_group(shapes, th, tw, dtype, nesterov, seed=10, mus=mus)
    g_np = [g.float().cpu().numpy() for g in grads]
    m_np = [m.float().cpu().numpy() for m in moms]
    grp.tiles.fill_(float("nan"))  # every element, padding included, must be written
    grp.gather()
    torch.cuda.synchronize()
    tiles = grp.tiles.float().cpu().numpy()
    ofs = 0
    for i, s in enumerate(shapes):
        ge, nb = O.momentum(g_np[i], m_np[i], mus[i], nesterov, dtype)
        assert np.array_equal(_bits(moms[i]), _bits(torch.from_numpy(nb).to(TDT[dtype]))), f"momentum param {i}"
        exp = _ns_layout(O.tile(O.bf16_round(ge), th, tw), grp.mp, grp.np)
        got = tiles[ofs : ofs + exp.shape[0]]
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), f"tiles param {i}"
        ofs += exp.shape[0]
    assert ofs == grp.n_tiles
    # per-tile norm and normaliser
    ssq = (tiles.astype(np.float64) ** 2).sum(axis=(1, 2))
    np.testing.assert_allclose(grp.partials.double().sum(1).cpu().numpy(), ssq, rtol=1e-5, atol=1e-30)
    inv = grp.inv.cpu().numpy()
    np.testing.assert_allclose(inv, 1.0 / (np.sqrt(ssq) + 1e-7), rtol=1e-5)


def test_gather_without_momentum_is_a_cast():
    grp, grads, _ = _make_group([(300, 700)], 256, 256, "float32", True, seed=3, with_mom=False)
    grp.gather()
    exp = _ns_layout(O.tile(O.bf16_round(grads[0].cpu().numpy()), 256, 256), grp.mp, grp.np)
    assert np.array_equal(grp.tiles.float().cpu().numpy(), exp)


@pytest.mark.parametrize("name,shapes,th,tw,dtype,nesterov", GATHER_CASES, ids=[c[0] for c in GATHER_CASES])
def test_untile_bit_exact(name, shapes, th, tw, dtype, nesterov):
    print(f"[untile] {name}", flush=True)
    grp, grads, _ = _make_group(shapes, th, tw, dtype, nesterov, seed=20)
    gen = torch.Generator().manual_seed(5)
    vals = torch.randn(grp.tiles.shape, generator=gen).to(torch.bfloat16)
    grp.tiles.copy_(vals.to(DEV))
    for u in grp.updates:
        u.fill_(float("nan"))
    grp.untile(steps=0)  # even step count: the result buffer is grp.tiles
    torch.cuda.synchronize()
    v = vals.float().numpy()
    ofs = 0
    scale = np.float32(O.lr_scale((th, tw)))
    for i, s in enumerate(shapes):
        R, Cc = O.tile_grid(s[0], s[1], th, tw)
        ns = v[ofs : ofs + R * Cc]
        t = ns[:, : min(th, tw), : max(th, tw)]
        t = np.swapaxes(t, 1, 2) if th > tw else t
        exp = O.round_to(O.untile(np.ascontiguousarray(t), s[0], s[1]) * scale, dtype)
        got = grp.updates[i].float().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), f"param {i}"
        ofs += R * Cc


# ---------------------------------------------------------------------------
# NS5
# ---------------------------------------------------------------------------
def _ns_engine(G: torch.Tensor, steps=5, family="auto") -> torch.Tensor:
    return newton_schulz(G, steps=steps, family=family)


NS_SHAPES = [
    # the reference's dispatch shapes (test_kernels.py:224-235)
    ("square_128", (4, 128, 128)),
    ("square_64", (8, 64, 64)),
    ("wide_64x256", (4, 64, 256)),
    ("wide_128x512", (4, 128, 512)),
    ("tall_128x64", (4, 128, 64)),
    ("big_512", (4, 512, 512)),
    ("2d_square_512", (512, 512)),
    ("2d_nondiv", (768, 513)),
    ("2d_tall", (513, 768)),
]


@pytest.mark.parametrize("label,shape", NS_SHAPES, ids=[s[0] for s in NS_SHAPES])
def test_newton_schulz_matches_reference_on_well_conditioned(label, shape, ns_family):
    """HiMuon.newton_schulz == the reference's NS in bf16 on well-conditioned
    inputs, with the reference test's elementwise tolerance (4e-2) and the
    north star's per-tile relative Frobenius bound (1e-2)."""
    print(f"[ns5 wc] {label} {shape} {ns_family}", flush=True)
    G = well_conditioned(shape, torch.bfloat16, seed=0)
    out = _ns_engine(G, family=ns_family)
    assert out.shape == G.shape and out.dtype == G.dtype
    assert torch.isfinite(out).all()
    ref_eager = ns5_torch_eager(G)
    assert torch.allclose(out.float(), ref_eager.float(), rtol=4e-2, atol=4e-2), label
    # a 2-D input takes the reference's 2-D third product (torch.addmm,
    # himuon.py:249-253), a batched one fused_bmm_add's
    ref = ns5_torch_staged(G, round_once=G.ndim == 2)
    err = per_tile_rel_fro(out, ref)
    print(f"  rel-fro vs staged torch: max {err.max():.4f} mean {err.mean():.4f}", flush=True)
    assert err.max() <= 1e-2, err


@pytest.mark.parametrize("T,n", [(128, 32), (256, 16), (512, 8)])
def test_ns5_random_tiles_vs_oracle_and_torch(T, n, ns_family):
    """Random (momentum-like) tiles: per-tile error against the torch
    same-dtype NS5 and the CPU oracle, next to the distance between those two
    references themselves (the summation-order noise floor of bf16 NS5)."""
    print(f"[ns5 random] T={T} n={n} {ns_family}", flush=True)
    G = _cpu_randn((n, T, T), seed=T, scale=1e-3).to(DEV)
    out = _ns_engine(G, family=ns_family)
    ref_t = ns5_torch_staged(G)
    ref_o = torch.from_numpy(O.ns5_staged(G.cpu().numpy())).to(DEV)
    e_t = per_tile_rel_fro(out, ref_t)
    e_o = per_tile_rel_fro(out, ref_o)
    floor = per_tile_rel_fro(ref_t, ref_o)
    print(f"  vs torch max {e_t.max():.4f} mean {e_t.mean():.4f} | vs oracle max {e_o.max():.4f} "
          f"mean {e_o.mean():.4f} | torch vs oracle max {floor.max():.4f} mean {floor.mean():.4f}", flush=True)
    # the north star's bar against the reference's NS5 in the same dtypes,
    # and bit-identity as built (same rounding points, same k order)
    assert e_t.max() <= 1e-2
    assert torch.equal(out, ref_t.to(out.dtype))
    # the numpy oracle sums in another order: bf16 NS5 amplifies that to the
    # noise floor the two references show against each other
    assert e_o.mean() <= 1e-2 and e_o.max() <= 2e-2
    assert e_o.mean() <= 1.5 * floor.mean() + 1e-3


@pytest.mark.parametrize("T,n", [(128, 16), (512, 4)])
def test_ns5_singular_value_band(T, n, ns_family):
    G = _cpu_randn((n, T, T), seed=T + 1, scale=1e-3).to(DEV)
    out = _ns_engine(G, family=ns_family).double()
    sv = torch.linalg.svdvals(out).cpu().numpy()
    ref_sv = torch.linalg.svdvals(ns5_torch_staged(G).double()).cpu().numpy()
    sv_in = torch.linalg.svdvals(G.double()).cpu().numpy()
    sv_in = sv_in / np.linalg.norm(G.double().cpu().numpy(), axis=(-2, -1))[:, None]
    floor, tol = 4e-3, 0.03
    for k in range(n):
        lo, hi = O.quintic_band(max(sv_in[k].min(), floor), sv_in[k].max())
        nn_ = int((sv_in[k] < floor).sum())
        assert sv[k].max() <= hi + tol and ref_sv[k].max() <= hi + tol
        assert (sv[k] < lo - tol).sum() <= nn_
        # same band as the reference: extremes agree
        assert abs(sv[k].max() - ref_sv[k].max()) < tol
        assert abs(np.sort(sv[k])[nn_] - np.sort(ref_sv[k])[nn_]) < 0.05


def test_ns5_zero_tile_and_padding(ns_family):
    # zero tiles map to zero (0 / (0 + eps) = 0); zero padding stays zero and
    # does not change the data block (a 37x100 block in a 256x256 tile equals
    # the same block NS'd in its own 128x128 padding, bit for bit, with the
    # 128-row kernels; AUTO runs a 37-row tile at 64 rows on 16 x 16 MFMA
    # tiles, another summation order: within the per-tile bar)
    G = torch.zeros(3, 256, 256, device=DEV)
    G[1, :37, :100] = _cpu_randn((37, 100), 4).to(DEV)
    out = _ns_engine(G, family=ns_family)
    assert (out[0] == 0).all() and (out[2] == 0).all()
    assert (out[1, 37:] == 0).all() and (out[1, :, 100:] == 0).all()
    blk = "block128" if ns_family == "auto" else ns_family
    small = _ns_engine(G[1:2, :37, :100].contiguous(), family=blk)
    assert torch.equal(out[1, :37, :100], small[0])
    if ns_family == "auto":
        few = _ns_engine(G[1:2, :37, :100].contiguous())
        assert per_tile_rel_fro(few, small).max() <= 1e-2


@pytest.mark.parametrize("shape", [(2, 256, 512), (2, 128, 128), (2, 128, 256), (2, 128, 512)],
                         ids=["256x512", "128", "128x256", "128x512"])
@pytest.mark.parametrize("steps", [0, 1, 2, 5])
def test_ns5_steps_honoured(steps, shape, ns_family):
    """Every step count, on the stream geometry and on the LDS-resident
    kernel's (which writes an even step count's result in place)."""
    G = _cpu_randn(shape, seed=9).to(DEV)
    out = _ns_engine(G, steps=steps, family=ns_family)
    ref = torch.from_numpy(O.ns5_staged(G.cpu().numpy(), steps=steps)).to(DEV)
    assert per_tile_rel_fro(out, ref).max() <= 1.5e-2
    assert torch.equal(out, ns5_torch_staged(G, steps=steps).to(out.dtype))


def test_ns5_sub_batch_invariance(ns_family):
    """Sub-batching (tiles are independent) does not change results bitwise."""
    G = _cpu_randn((10, 256, 256), seed=12, scale=1e-3).to(DEV)
    grp = TileGroup([G.view(-1, 256)], [G.view(-1, 256)], [None], 256, 256, [1.0], [0.0], [False],
                    torch.device(DEV), torch.float32, ns_family=ns_family)
    outs = []
    for sb in (1, 3, 10):
        grp.gather()  # NS overwrites both X orientations (ping-pong): re-gather each run
        ws = torch.empty(grp.workspace_bytes(sb), device=DEV, dtype=torch.uint8)
        grp.ns(0, grp.n_tiles, 5, ws, sb)
        outs.append(grp.result(5).clone())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


STALE_SHAPES = [
    # (label, n, M, N): one per kernel family / geometry class
    ("lds_128", 3, 128, 128),
    ("lds_100x200", 3, 100, 200),
    ("lds_100x400", 3, 100, 400),
    ("blk_100x300", 3, 100, 300),
    ("blk_tall_300x100", 3, 300, 100),
    ("blk_300x300", 2, 300, 300),
    ("stream_256", 3, 256, 256),
    ("stream_200x500", 2, 200, 500),
    ("stream_tall_1000x400", 2, 1000, 400),
    ("few_rows_16x1024", 3, 16, 1024),
    ("few_rows_tall_300x40", 2, 300, 40),
]


@pytest.mark.parametrize("label,n,M,N", STALE_SHAPES, ids=[s[0] for s in STALE_SHAPES])
def test_ns5_ignores_stale_buffer_contents(label, n, M, N, ns_family):
    """The tile buffers and the NS workspace come from torch.empty: every
    element any kernel reads must have been written earlier in the same step.
    NaN-filled buffers must give bit-for-bit the result of zero-filled ones."""
    print(f"[ns5 stale] {label} {ns_family}", flush=True)
    G = _cpu_randn((n, M, N), seed=M + N, scale=1e-3).to(torch.bfloat16).to(DEV)
    outs = []
    for fill in (0.0, float("nan")):
        flat = G.reshape(-1, N)
        grp = TileGroup([flat], [flat], [None], M, N, [1.0], [0.0], [False], torch.device(DEV), torch.bfloat16,
                        ns_family=ns_family)
        sb = grp.default_sub_batch()
        ws = torch.empty(max(2, grp.workspace_bytes(sb)), device=DEV, dtype=torch.uint8)
        grp.tiles.fill_(fill)
        grp.alt.fill_(fill)
        ws.view(torch.bfloat16).fill_(fill)
        grp.updates[0].fill_(fill)
        grp.gather()
        grp.ns(0, grp.n_tiles, 5, ws, sb)
        grp.untile(5)
        outs.append(grp.updates[0].clone())
    assert torch.isfinite(outs[1].float()).all()
    assert torch.equal(outs[0], outs[1])
    err = per_tile_rel_fro(outs[1].view(n, M, N).float(), ns5_torch_staged(G).float())
    assert err.max() <= 1e-2, err


def test_ns5_workspace_too_small_raises():
    G = _cpu_randn((2, 128, 128), seed=1).to(DEV)
    grp = TileGroup([G.view(-1, 128)], [G.view(-1, 128)], [None], 128, 128, [1.0], [0.0], [False],
                    torch.device(DEV), torch.float32)
    grp.gather()
    ws = torch.empty(16, device=DEV, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="workspace"):
        grp.ns(0, 2, 5, ws, 2)


def test_ns5_many_tiles_large_buffers():
    """4096 tiles of 512x512: tile buffers of 2 GiB (addresses with bit 31 of
    the low word set, as for real models), persistent workgroups that run many
    output blocks each (cross-block operand prefetch and deferred stores).
    Sampled tiles match the reference's same-dtype NS5; the result does not
    depend on the sub-batch size (bitwise)."""
    n, T = 4096, 512
    print(f"[ns5 large] n={n}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(7)
    G = (torch.randn((n, T, T), generator=gen, device=DEV) * 1e-3).to(torch.bfloat16)
    flat = G.view(-1, T)
    grp = TileGroup([flat], [flat], [None], T, T, [1.0], [0.0], [False], torch.device(DEV), torch.bfloat16)
    outs = []
    for sb in (n, 1000):
        grp.gather()
        ws = torch.empty(grp.workspace_bytes(sb), device=DEV, dtype=torch.uint8)
        grp.ns(0, grp.n_tiles, 5, ws, sb)
        outs.append(grp.result(5).clone())
        del ws
    assert torch.equal(outs[0], outs[1])
    out = outs[0]
    assert torch.isfinite(out.float()).all()
    idx = torch.tensor([0, 1, 2, 1023, 2048, 2049, 3071, 4095], device=DEV)
    ref = ns5_torch_staged(G[idx])
    err = per_tile_rel_fro(out[idx].float(), ref.float())
    print(f"  sampled tiles vs staged torch: max {err.max():.4f} mean {err.mean():.4f}", flush=True)
    assert err.max() <= 1e-2
    assert torch.equal(out[idx], ref)


FEW_ROWS = [(8, 16, 1024), (4, 32, 512), (4, 64, 128), (6, 16, 128), (3, 1, 300), (2, 5, 2048), (2, 48, 100),
            (3, 20, 640), (2, 32, 1024), (2, 1024, 16), (16, 1024), (4, 64, 256)]


@pytest.mark.parametrize("shape", FEW_ROWS, ids=["x".join(map(str, s)) for s in FEW_ROWS])
@pytest.mark.parametrize("steps", [1, 2, 5])
def test_ns5_few_rows(shape, steps):
    """NS operands of m <= 64 rows iterate at 16, 32 or 64 rows (HIMUON_NS_ROWS;
    the reference's small-M shapes, himuon.py:261-284), on 16 x 16 MFMA tiles,
    one workgroup per tile. Against torch's same-dtype NS5: per-tile relative
    Frobenius <= 1e-2 (the north star's bar; another summation order than
    torch's, so not bit for bit), as the 128-row kernels on the padded tiles;
    against the numpy oracle at the noise floor; singular values in
    the quintic's band. Odd and even step counts (result in either buffer), a
    tall input (transposed) and a 2-D one (the addmm rounding)."""
    print(f"[ns5 few rows] {shape} steps={steps}", flush=True)
    G = _cpu_randn(shape, seed=sum(shape) + steps, scale=1e-3).to(DEV)
    out = newton_schulz(G, steps=steps)
    ref = ns5_torch_staged(G, steps=steps, round_once=G.ndim == 2)
    blk = newton_schulz(G, steps=steps, family="block128")  # all 128 padded rows
    assert out.shape == G.shape and torch.isfinite(out).all()
    err = per_tile_rel_fro(out, ref)
    assert per_tile_rel_fro(blk, ref).max() <= 1e-2
    ref_o = O.ns5_staged_2d(G.cpu().numpy(), steps=steps) if G.ndim == 2 else O.ns5_staged(G.cpu().numpy(), steps=steps)
    e_o = per_tile_rel_fro(out, torch.from_numpy(ref_o).to(DEV))
    print(f"  vs torch max {err.max():.2e}, vs oracle max {e_o.max():.2e}", flush=True)
    assert err.max() <= 1e-2
    assert e_o.mean() <= 1e-2 and e_o.max() <= 2e-2
    if steps == 5:
        g3 = G.reshape(-1, *G.shape[-2:]).double()
        sv = torch.linalg.svdvals(out.reshape(g3.shape).double()).cpu().numpy()
        sv_in = torch.linalg.svdvals(g3).cpu().numpy()
        sv_in = sv_in / np.linalg.norm(g3.cpu().numpy(), axis=(-2, -1))[:, None]
        for k in range(sv.shape[0]):
            lo, hi = O.quintic_band(max(sv_in[k].min(), 4e-3), sv_in[k].max())
            assert sv[k].max() <= hi + 0.03 and sv[k].min() >= lo - 0.03


def test_newton_schulz_replays_and_captures():
    """newton_schulz keeps its device state per shape and replays a graph of
    its launches per step count: consecutive calls with new inputs (and
    another step count) equal the launches run eagerly on the same inputs,
    the inputs are not modified, each call returns a new tensor; and the call
    can itself be recorded into a caller's graph and replayed."""
    from himuon_amd import engine as E

    shape = (6, 256, 512)
    gs = [_cpu_randn(shape, seed=70 + k, scale=1e-3).to(DEV) for k in range(3)]
    keep = [g.clone() for g in gs]
    outs = [newton_schulz(gs[0]), newton_schulz(gs[1]), newton_schulz(gs[2], steps=3), newton_schulz(gs[0])]
    for g, k in zip(gs, keep):
        assert torch.equal(g, k)
    assert outs[0].data_ptr() != outs[3].data_ptr() and torch.equal(outs[0], outs[3])
    for out, g, st in zip(outs, (gs[0], gs[1], gs[2]), (5, 5, 3)):
        plan = E._NsPlan(shape[0], shape[1], shape[2], torch.float32, g.device, False, "auto")
        plan.xin.view(shape).copy_(g)
        plan._launches(st)
        assert torch.equal(out, plan.out.view(shape))
    # recorded into a caller's capture (launches, not a nested replay)
    static_in = gs[1].clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_out = newton_schulz(static_in)
    for k in range(3):
        static_in.copy_(gs[k])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out, newton_schulz(gs[k]))
