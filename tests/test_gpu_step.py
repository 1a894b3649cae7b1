"""GPU behaviour of HiMuon.step() on the HIP path.

Step-level parity against the CPU oracle (oracle.step_param), bit-exact
momentum buffers, self-consistency (b_hw chunking, eager vs hipGraph replay,
reconfigure to the same tile), plan/dispatch accounting, cache invalidation,
peak-memory stability and a smoke matrix — the behaviours the reference pins
in tests/integration/test_himuon_{self_consistency,dispatch,reconfigure,
memory,smoke}.py.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch
import torch.nn as nn

from oracle import himuon_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from himuon_amd.optimizers.himuon import HiMuon

    from gpu_ref import ns5_torch_staged

DEV = "cuda"
RTOL = ATOL = 1e-2  # reference self-consistency tolerance (test_himuon_self_consistency.py:18)


def make_model(shapes, dtype=torch.float32, bias=False, seed=0):
    torch.manual_seed(seed)
    layers = [nn.Linear(w, h, bias=bias, dtype=dtype) for (h, w) in shapes]
    return nn.ModuleList(layers).to(DEV)


def muon_groups(model, wd=0.0, **extra):
    muon = [p for p in model.parameters() if p.ndim >= 2]
    one_d = [p for p in model.parameters() if p.ndim < 2]
    groups = [{"params": muon, "weight_decay": wd, "use_muon": True, **extra}]
    if one_d:
        groups.append({"params": one_d, "lr": 1e-3, "weight_decay": 0.0, "use_muon": False})
    return groups


def seed_grads(model, seed):
    """Fill grads in place (stable pointers), from a CPU generator."""
    g = torch.Generator().manual_seed(seed)
    for p in model.parameters():
        vals = torch.randn(p.shape, generator=g).to(p.dtype)
        if p.grad is None:
            p.grad = torch.empty_like(p)
        p.grad.copy_(vals.to(DEV))


def _np(t):
    return t.detach().float().cpu().numpy()


# ---------------------------------------------------------------------------
# Parity against the oracle
# ---------------------------------------------------------------------------
STEP_CASES = [
    ("fp32_T256", [(512, 1024), (256, 512), (1024, 2048)], 256, torch.float32),
    ("bf16_T512_pad", [(768, 513), (512, 1024)], 512, torch.bfloat16),
    ("fp32_tall_tiles", [(384, 256)], (128, 64), torch.float32),
    ("full_ns_mix", [(64, 64), (256, 1024), (100, 40)], 512, torch.float32),
]


@pytest.mark.parametrize("name,shapes,tile,dtype", STEP_CASES, ids=[c[0] for c in STEP_CASES])
def test_step_matches_oracle(name, shapes, tile, dtype):
    print(f"[step vs oracle] {name}", flush=True)
    lr, wd, steps = 0.02, 0.1, 3
    model = make_model(shapes, dtype)
    opt = HiMuon(muon_groups(model, wd=wd), lr=lr, tile_size=tile, cuda_graph=False)
    ts = opt.param_groups[0]["tile_size"]
    p_np = [_np(p) for p in model.parameters()]
    bufs = [None] * len(p_np)
    dname = "bfloat16" if dtype == torch.bfloat16 else "float32"
    for k in range(steps):
        seed_grads(model, 100 + k)
        g_np = [_np(p.grad) for p in model.parameters()]
        prev = [_np(p) for p in model.parameters()]
        opt.step()
        for i, p in enumerate(model.parameters()):
            op = O.OracleParam(p=p_np[i], g=g_np[i], buf=bufs[i], tile=ts, lr=lr, wd=wd,
                               p_dtype=dname, g_dtype=dname)
            p_np[i], bufs[i], _ = O.step_param(op)
            if dtype != torch.float32:
                # bf16 parameters: this step from the GPU's own previous
                # parameters and momentum, with the oracle's momentum, tiling,
                # untiling, scale and WD/LR roundings around torch's
                # same-dtype NS5 on the GPU, which the library's NS5 equals bit
                # for bit: the new parameters must match bit for bit (the
                # numpy NS5's summation order would move single bf16 roundings)
                def torch_ns(x, steps):
                    t = torch.from_numpy(x).to(DEV)
                    return ns5_torch_staged(t, steps, round_once=x.ndim == 2).float().cpu().numpy()

                op_gpu = O.OracleParam(p=prev[i], g=g_np[i], buf=None if k == 0 else bufs_prev[i], tile=ts,
                                       lr=lr, wd=wd, p_dtype=dname, g_dtype=dname)
                exp_p, _, _ = O.step_param(op_gpu, ns=torch_ns)
                got = _np(p)
                assert np.array_equal(got, exp_p), (name, i, k, int((got != exp_p).sum()), got.size)
                continue
            # this step's update, per NS tile, from the GPU's own previous
            # parameters: relative Frobenius error at the noise floor of
            # differently ordered bf16 NS5 (a wrong term or scale is O(1))
            op_gpu = O.OracleParam(p=prev[i], g=g_np[i], buf=None if k == 0 else bufs_prev[i], tile=ts,
                                   lr=lr, wd=wd, p_dtype=dname, g_dtype=dname)
            exp_p, _, _ = O.step_param(op_gpu)
            base = prev[i] * np.float32(1 - lr * wd)
            d_got, d_exp = _np(p) - base, exp_p - base
            h, w = d_exp.shape
            th, tw = (h, w) if h * w <= ts[0] * ts[1] else ts
            errs = []
            for r0 in range(0, h, th):
                for c0 in range(0, w, tw):
                    sl = (slice(r0, r0 + th), slice(c0, c0 + tw))
                    errs.append(np.linalg.norm(d_got[sl] - d_exp[sl]) / np.linalg.norm(d_exp[sl]))
            errs = np.array(errs)
            assert errs.max() <= 2e-2 and errs.mean() <= 1e-2, (name, i, k, errs.max(), errs.mean())
        bufs_prev = list(bufs)
    for i, p in enumerate(model.parameters()):
        buf = opt.state[p]["momentum_buffer"]
        assert np.array_equal(_np(buf), bufs[i]), f"momentum buffer {i} not bit-exact"
        np.testing.assert_allclose(_np(p), p_np[i], rtol=RTOL, atol=ATOL)
        assert np.isfinite(_np(p)).all()


def test_update_tensor_matches_oracle_per_tile():
    """The update tensor (non-fused untile) of one param vs the oracle's, per
    tile (relative Frobenius), bit-exact momentum."""
    from himuon_amd.engine import TileGroup

    shapes, T = [(1024, 1536)], 512
    model = make_model(shapes, torch.float32)
    seed_grads(model, 7)
    p = model[0].weight
    g = _np(p.grad)
    mom = torch.zeros_like(p.grad)
    grp = TileGroup(params=[p], grads=[p.grad], moms=[mom], tile_h=T, tile_w=T,
                    upd_scales=[float(O.lr_scale((T, T)))], mus=[0.95], nesterovs=[True],
                    device=p.device, dtype=torch.float32)
    ws = torch.empty(grp.workspace_bytes(grp.default_sub_batch()), device=DEV, dtype=torch.uint8)
    grp.gather()
    grp.ns(0, grp.n_tiles, 5, ws, grp.default_sub_batch())
    grp.untile(5)
    ge, nb = O.momentum(g, np.zeros_like(g), 0.95, True)
    assert np.array_equal(_np(mom), nb)
    ref = O.untile(O.ns5_staged(O.tile(ge, T, T)), *shapes[0]) * np.float32(O.lr_scale((T, T)))
    got = _np(grp.updates[0])
    for r in range(2):
        for c in range(3):
            sl = (slice(r * T, (r + 1) * T), slice(c * T, (c + 1) * T))
            e = np.linalg.norm(got[sl] - ref[sl]) / np.linalg.norm(ref[sl])
            assert e < 2e-2, (r, c, e)


@pytest.mark.parametrize("pdt", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("cuda_graph", [False, True])
@pytest.mark.parametrize("tile", [256, (512, 256), 512, 128])
def test_fused_untile_apply_matches_unfused(pdt, cuda_graph, tile):
    """The fused untile (WD/LR applied in place, inside the graph) leaves the
    parameters bit-identical to the unfused path (update tensors, then the
    WD/LR pass), over several steps with an lr/wd change between steps, which
    the fused path reads from its device table without a recapture. Three
    param groups with their own lr/wd; wide, square and tall tiles (the
    transposed untile), ragged edges and full-matrix NS groups."""
    shapes = [(512, 1024), (256, 512), (700, 300), (300, 100), (100, 300), (1024, 512)]
    settings = [(0.02, 0.05), (0.01, 0.0), (0.03, 0.2)]
    m_f = make_model(shapes, pdt)
    m_u = copy.deepcopy(m_f)

    def groups(m):
        ps = list(m.parameters())
        return [{"params": ps[2 * i: 2 * i + 2], "lr": lr, "weight_decay": wd, "use_muon": True}
                for i, (lr, wd) in enumerate(settings)]

    m_r = copy.deepcopy(m_f)
    kw = dict(tile_size=tile, cuda_graph=cuda_graph, cuda_graph_warmup=2)
    o_f = HiMuon(groups(m_f), **kw)
    o_u = HiMuon(groups(m_u), **kw)
    o_u._fuse_untile = False
    # referee: eager, unfused (WD/LR by the reference's torch ops)
    o_r = HiMuon(groups(m_r), **{**kw, "cuda_graph": False})
    o_r._fuse_untile = False
    runs = ((m_f, o_f), (m_u, o_u), (m_r, o_r))
    for k in range(7):
        if k == 5:
            for _, o in runs:
                o.param_groups[0]["lr"] = 0.01
                o.param_groups[0]["weight_decay"] = 0.1
                o.param_groups[2]["weight_decay"] = 0.0
        for m, o in runs:
            seed_grads(m, 400 + k)
            o.step()
    assert all(g["tiles"].fused for g in o_f._groups)
    assert not any(g["tiles"].fused for g in o_u._groups)
    if tile != 128:  # (at 128 every matrix is tiled: no tall whole-matrix group)
        assert any(g["tiles"].tile_h > g["tiles"].tile_w for g in o_f._groups)  # transposed untile ran
    # 128 x 128 NS tiles of fp32/bf16 parameters: the whole step ran in LDS
    assert any(g["tiles"].lds_step_ok() for g in o_f._groups) == (tile == 128 and pdt != torch.float16)
    if cuda_graph:
        assert o_f._cuda_graph is not None and o_f._pending_updates
        assert all(u is None for _, u, _ in o_f._pending_updates)
    def diffs(m, ref):
        out = []
        for i, (a, r) in enumerate(zip(m.parameters(), ref.parameters())):
            if not torch.equal(a, r):
                out.append((i, tuple(a.shape), int((a != r).sum()), a.numel(),
                            float((a.detach().float() - r.detach().float()).abs().max())))
        return out

    if pdt == torch.float16:
        # torch's fp16 p.add_(u, alpha=-lr) is p + alpha*u as one fp32 fma (the form
        # the kernels use) in its vectorised bulk path, measured bit for bit on the
        # GPU, but not in the non-vectorised tail of each launch (the last
        # partial block, up to a few thousand elements), which rounds some
        # elements differently by 1 ulp. The tail covers the same elements every
        # step, so over 7 steps those drift by a few ulp. Against torch's ops (the
        # referee, and the unfused path's eager warm-up steps): at most 0.1 % of
        # the elements plus 100 (a small matrix is mostly tail), by at most 1e-3
        # (parameters ~0.05).
        for name, m in (("fused", m_f), ("unfused", m_u)):
            for i, shape, n_bad, n, dmax in diffs(m, m_r):
                assert n_bad <= 1e-3 * n + 100 and dmax <= 1e-3, (name, i, shape, n_bad, dmax)
        return
    bad = [("fused",) + d for d in diffs(m_f, m_r)] + [("unfused",) + d for d in diffs(m_u, m_r)]
    assert not bad, bad


# ---------------------------------------------------------------------------
# Self-consistency (test_himuon_self_consistency.py)
# ---------------------------------------------------------------------------
SHAPES = [(512, 1024), (256, 512), (1024, 2048)]


def test_result_invariant_to_b_hw():
    kw = dict(lr=0.02, weight_decay=0.1, tile_size=512, ns_steps=5, cuda_graph=False)
    m_big = make_model(SHAPES, torch.bfloat16)
    m_small = copy.deepcopy(m_big)
    o_big = HiMuon(muon_groups(m_big, wd=0.1), b_hw=100_000, **kw)
    o_small = HiMuon(muon_groups(m_small, wd=0.1), b_hw=1, **kw)
    for k in range(5):
        seed_grads(m_big, 100 + k)
        seed_grads(m_small, 100 + k)
        o_big.step()
        o_small.step()
    for a, b in zip(m_big.parameters(), m_small.parameters()):
        assert torch.equal(a, b)  # tiles are independent: chunking is exact


def test_eager_matches_graph():
    kw = dict(lr=0.02, weight_decay=0.05, tile_size=512, ns_steps=5)
    m_e = make_model(SHAPES, torch.bfloat16)
    m_g = copy.deepcopy(m_e)
    o_e = HiMuon(muon_groups(m_e, wd=0.05), cuda_graph=False, **kw)
    o_g = HiMuon(muon_groups(m_g, wd=0.05), cuda_graph=True, cuda_graph_warmup=3, **kw)
    for k in range(8):
        seed_grads(m_e, 200 + k)
        seed_grads(m_g, 200 + k)
        o_e.step()
        o_g.step()
    assert o_g._cuda_graph is not None
    for a, b in zip(m_e.parameters(), m_g.parameters()):
        assert torch.equal(a, b)


def test_fp16_params_fp32_grads_eager_matches_graph():
    """fp16 parameters with fp32 grads: the update stays fp32 and is not
    fused into the untile; eagerly the reference's torch ops add it, under
    replay the HIP WD/LR pass does, rounding p + alpha * u once from the exact
    value as torch's mixed-dtype add does over a large tensor: bit-identical
    for the 512 x 1024 parameter. torch takes other rounding forms on smaller
    tensors (measured: 0.8 % and 6 % of the elements of the 700 x 300 and
    300 x 100 parameters, 1 ulp), bounded here."""
    shapes = [(512, 1024), (700, 300), (300, 100)]
    gen = torch.Generator().manual_seed(5)
    base = [(torch.randn(*s, generator=gen) * 0.02).half() for s in shapes]

    def params():
        ps = []
        for b in base:
            p = torch.nn.Parameter(b.clone().to(DEV))
            p.grad_dtype = torch.float32
            ps.append(p)
        return ps

    def groups(ps):
        return [{"params": ps[:1], "lr": 0.02, "weight_decay": 0.1, "use_muon": True},
                {"params": ps[1:], "lr": 0.01, "weight_decay": 0.05, "use_muon": True}]

    p_e, p_g = params(), params()
    o_e = HiMuon(groups(p_e), tile_size=256, cuda_graph=False)
    o_g = HiMuon(groups(p_g), tile_size=256, cuda_graph=True, cuda_graph_warmup=2)
    for k in range(6):
        g = torch.Generator().manual_seed(300 + k)
        for a, b in zip(p_e, p_g):
            v = (torch.randn(a.shape, generator=g) * 1e-3).to(DEV)
            for p in (a, b):
                if p.grad is None:
                    p.grad = torch.empty_like(v)
                p.grad.copy_(v)
        o_e.step()
        o_g.step()
    assert o_g._cuda_graph is not None
    assert not any(grp["tiles"].fused for grp in o_g._groups)
    assert all(grp["tiles"].upd_dtype == torch.float32 for grp in o_g._groups)
    rep = [(tuple(a.shape), int((a != b).sum()), a.numel(), float((a.detach().float() - b.detach().float()).abs().max()))
           for a, b in zip(p_e, p_g)]
    for a, b in zip(p_e, p_g):
        assert a.dtype == torch.float16
        if a.numel() >= 1 << 19:
            assert torch.equal(a, b), rep
        else:
            assert (a.float() - b.float()).abs().max() <= 1.3e-4, rep  # 1-2 fp16 ulp at |p| < 0.1


def test_graph_replays_track_lr_schedule():
    """LR/WD are read outside the graph: changing group lr between replays
    takes effect without recapture."""
    m_e = make_model([(512, 1024)], torch.float32)
    m_g = copy.deepcopy(m_e)
    o_e = HiMuon(muon_groups(m_e, wd=0.1), tile_size=256, cuda_graph=False)
    o_g = HiMuon(muon_groups(m_g, wd=0.1), tile_size=256, cuda_graph=True, cuda_graph_warmup=1)
    for k in range(6):
        for o in (o_e, o_g):
            o.param_groups[0]["lr"] = 0.02 * (k + 1) / 6
        seed_grads(m_e, 300 + k)
        seed_grads(m_g, 300 + k)
        o_e.step()
        o_g.step()
    for a, b in zip(m_e.parameters(), m_g.parameters()):
        assert torch.equal(a, b)


# ---------------------------------------------------------------------------
# Dispatch / plan (test_himuon_dispatch.py)
# ---------------------------------------------------------------------------
MULTI = [(512, 1024), (256, 512), (1024, 2048)]


def test_every_tile_accounted_for():
    T = 256
    model = make_model(MULTI, bias=True)
    opt = HiMuon(muon_groups(model), tile_size=T, cuda_graph=False)
    seed_grads(model, 12)
    opt.step()
    counts = {}
    for b in opt.xlayer_plan():
        for pid, tc in zip(b["param_ids"], b["tile_count_per_param"]):
            counts[pid] = counts.get(pid, 0) + tc
    for p in model.parameters():
        if p.ndim < 2:
            continue
        exp = (-(-p.shape[0] // T)) * (-(-p.shape[1] // T))
        if id(p) in counts:
            assert counts[id(p)] == exp
        else:
            assert p.numel() <= T * T
    assert opt._last_step_stats["ns_launches"] >= 1


def test_chunks_and_override():
    model = make_model(MULTI)
    opt = HiMuon(muon_groups(model), tile_size=512, cuda_graph=False)
    seed_grads(model, 14)
    opt.step()
    for b in opt.xlayer_plan():
        assert sum(b["chunk_sizes"]) == b["B_total"] and all(0 < c <= b["B_hw"] for c in b["chunk_sizes"])
        assert b["n_calls"] == len(b["chunk_sizes"])
    B_total = max(b["B_total"] for b in opt.xlayer_plan())
    for b_hw, n_expect in ((B_total + 10, 1), (B_total, 1), (max(1, B_total // 2), -(-B_total // max(1, B_total // 2)))):
        m = make_model(MULTI)
        o = HiMuon(muon_groups(m), tile_size=512, b_hw=b_hw, cuda_graph=False)
        seed_grads(m, 19)
        o.step()
        assert o.xlayer_plan()[0]["n_calls"] == n_expect
    m = make_model([(1024, 1024)])
    o = HiMuon(muon_groups(m), tile_size=512, b_hw=7, cuda_graph=False)
    seed_grads(m, 22)
    o.step()
    assert o.xlayer_plan()[0]["B_hw"] == 7


# ---------------------------------------------------------------------------
# Reconfigure (test_himuon_reconfigure.py)
# ---------------------------------------------------------------------------
def test_reconfigure_invalidates_and_takes_effect():
    model = make_model([(512, 1024)], torch.bfloat16)
    opt = HiMuon(muon_groups(model), tile_size=512, cuda_graph=True, cuda_graph_warmup=2)
    for k in range(4):
        seed_grads(model, 10 + k)
        opt.step()
    assert opt._cuda_graph is not None and opt._pending_updates and opt.xlayer_plan() and opt._concat_buffers
    opt.reconfigure(tile_size=256)
    assert opt._cuda_graph is None and opt._graph_step_count == 0 and opt._pending_updates == []
    assert opt.xlayer_plan() == [] and opt._concat_buffers == {}
    seed_grads(model, 20)
    opt.step()
    assert {(b["bucket_key"][0], b["bucket_key"][1]) for b in opt.xlayer_plan()} == {(256, 256)}


@pytest.mark.parametrize("cuda_graph", [False, True])
def test_reconfigure_same_tile_is_noop(cuda_graph):
    shapes, K = [(512, 1024), (256, 512)], 6
    ref = make_model(shapes, torch.bfloat16)
    rec = copy.deepcopy(ref)
    kw = dict(lr=0.02, weight_decay=0.05, tile_size=256, cuda_graph=cuda_graph, cuda_graph_warmup=2)
    o_ref = HiMuon(muon_groups(ref, wd=0.05), **kw)
    o_rec = HiMuon(muon_groups(rec, wd=0.05), **kw)
    for k in range(2 * K):
        seed_grads(ref, 200 + k)
        seed_grads(rec, 200 + k)
        o_ref.step()
        if k == K:
            o_rec.reconfigure(tile_size=256)
        o_rec.step()
    for a, b in zip(ref.parameters(), rec.parameters()):
        assert torch.equal(a, b)


def test_reconfigure_128_to_512_recaptures():
    """Small-tile regime then a mid-run reconfigure to 512 (graph recapture)."""
    model = make_model([(1024, 1024), (512, 2048)], torch.float32)
    opt = HiMuon(muon_groups(model, wd=0.1), tile_size=128, cuda_graph=True, cuda_graph_warmup=1)
    for k in range(3):
        seed_grads(model, k)
        opt.step()
    assert opt.xlayer_plan()[0]["B_total"] == 64 + 64
    g1 = opt._cuda_graph
    opt.reconfigure(tile_size=512)
    for k in range(3):
        seed_grads(model, 10 + k)
        opt.step()
    assert opt._cuda_graph is not None and opt._cuda_graph is not g1
    assert opt.xlayer_plan()[0]["B_total"] == 4 + 4
    assert all(torch.isfinite(p).all() for p in model.parameters())


# ---------------------------------------------------------------------------
# Memory (test_himuon_memory.py) and smoke (test_himuon_smoke.py)
# ---------------------------------------------------------------------------
def test_no_peak_memory_growth():
    model = make_model([(1024, 1024), (512, 2048)])
    opt = HiMuon(muon_groups(model, wd=0.1), tile_size=512)
    for i in range(8):
        seed_grads(model, 300 + i)
        opt.step()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    peaks = []
    for i in range(10):
        torch.cuda.reset_peak_memory_stats()
        seed_grads(model, 400 + i)
        opt.step()
        torch.cuda.synchronize()
        peaks.append(torch.cuda.max_memory_allocated())
    assert (max(peaks) - min(peaks)) / max(min(peaks), 1) < 0.01, peaks


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("tile", [128, 256, 512])
def test_smoke_finite_and_changed(dtype, tile):
    model = make_model([(512, 1024), (768, 513), (64, 64)], dtype, bias=True)
    opt = HiMuon(muon_groups(model), tile_size=tile, cuda_graph=False)
    before = [p.detach().clone() for p in model.parameters()]
    seed_grads(model, 1)
    opt.step()
    assert all(torch.isfinite(p).all() for p in model.parameters())
    assert any(not torch.equal(p, b) for p, b in zip(model.parameters(), before))


def test_closure_and_cuda_graph_mode_runs():
    model = make_model([(512, 1024)])
    opt = HiMuon(muon_groups(model), tile_size=512, cuda_graph=True, cuda_graph_warmup=2)
    for k in range(5):
        seed_grads(model, 20 + k)
        assert opt.step(closure=lambda: 1.5) == 1.5
    assert opt._cuda_graph is not None
    assert all(torch.isfinite(p).all() for p in model.parameters())


@pytest.mark.parametrize("cuda_graph", [False, True])
def test_grad_set_changes_rebuild_the_step(cuda_graph):
    """A small (full-matrix) parameter without a grad on a step is skipped, and
    updated again once it has one (the reference scans full-matrix parameters
    every step, himuon.py:846-858); a tiled parameter likewise. In graph mode
    the change drops the graph: warm-up and recapture follow."""
    model = make_model([(256, 512), (64, 64), (512, 1024)], torch.float32)
    opt = HiMuon(muon_groups(model, wd=0.1), lr=0.02, tile_size=256, cuda_graph=cuda_graph,
                 cuda_graph_warmup=1)
    small, big = model[1].weight, model[2].weight
    for k in range(3):
        seed_grads(model, 200 + k)
        opt.step()
    torch.cuda.synchronize()
    if cuda_graph:
        assert opt._cuda_graph is not None
    # step 4: the small and the big parameter lose their grads
    frozen = {id(p): p.detach().clone() for p in (small, big)}
    buf_small = opt.state[small]["momentum_buffer"].clone()
    small.grad = None
    big.grad = None
    opt.step()
    torch.cuda.synchronize()
    assert torch.equal(small.detach(), frozen[id(small)]) and torch.equal(big.detach(), frozen[id(big)])
    assert torch.equal(opt.state[small]["momentum_buffer"], buf_small)
    # step 5: both have grads again (new storage): updated with the momentum kept
    seed_grads(model, 300)
    p_before = small.detach().clone()
    g = _np(small.grad)
    opt.step()
    opt.step() if cuda_graph else None  # graph mode: the warm-up step, then capture + replay
    torch.cuda.synchronize()
    assert not torch.equal(small.detach(), p_before)
    n = 2 if cuda_graph else 1
    buf = _np(buf_small)
    for _ in range(n):
        _, buf = O.momentum(g, buf, 0.95, True)
    assert np.array_equal(_np(opt.state[small]["momentum_buffer"]), buf)
    if cuda_graph:
        assert opt._cuda_graph is not None


@pytest.mark.parametrize("cuda_graph", [False, True])
def test_param_storage_change_is_followed(cuda_graph):
    """p.data reassigned between steps (e.g. by checkpoint loading): the next
    step updates the new storage, never the old one (the device tables and a
    captured graph hold parameter pointers)."""
    model = make_model([(512, 512)], torch.float32)
    opt = HiMuon(muon_groups(model, wd=0.1), lr=0.02, tile_size=256, cuda_graph=cuda_graph,
                 cuda_graph_warmup=1)
    p = model[0].weight
    for k in range(3):
        seed_grads(model, 400 + k)
        opt.step()
    torch.cuda.synchronize()
    old = p.data
    old_copy = old.clone()
    p.data = old.clone() * 0.5  # new storage
    new_before = p.detach().clone()
    opt.step()
    torch.cuda.synchronize()
    assert torch.equal(old, old_copy), "the old parameter storage was written"
    assert not torch.equal(p.detach(), new_before), "the new parameter storage was not updated"


@pytest.mark.parametrize("cuda_graph", [False, True])
def test_fresh_grads_every_step_keep_the_device_state(cuda_graph):
    """zero_grad(set_to_none=True) between steps (train.py --no-cuda-graph,
    train_fsdp.py): every backward allocates new grads. The plan and tile
    groups stay the same objects (only the descriptor tables are rewritten, in
    place), no old grad is kept alive, and the parameters equal those of a run
    whose grads are filled in place, bit for bit. In graph mode the moved
    grads drop the captured graph (never replayed on stale pointers), which
    is then warmed up and recaptured. The previous grads stay referenced here
    until the new ones exist, so the new ones cannot reuse their memory."""
    shapes = [(512, 1024), (256, 512), (1024, 512), (64, 64)]
    m_a = make_model(shapes, torch.bfloat16, bias=True)
    m_b = copy.deepcopy(m_a)
    kw = dict(lr=0.02, weight_decay=0.1, tile_size=256, cuda_graph=cuda_graph, cuda_graph_warmup=2)
    o_a = HiMuon(muon_groups(m_a, wd=0.1), **kw)
    o_b = HiMuon(muon_groups(m_b, wd=0.1), **kw)
    groups = None
    for k in range(6):
        seed_grads(m_a, 500 + k)
        o_a.step()
        old = [p.grad for p in m_b.parameters()]
        for p in m_b.parameters():
            p.grad = None  # zero_grad(set_to_none=True)
        seed_grads(m_b, 500 + k)  # fresh grad tensors
        if k >= 1:
            assert all(p.grad.data_ptr() != o.data_ptr() for p, o in zip(m_b.parameters(), old))
        del old
        o_b.step()
        if k >= 1:
            assert o_b._groups is groups, "tile groups rebuilt for fresh grads"
        groups = o_b._groups
        for g in o_b._groups:
            assert g["tiles"]._bound is None  # the step kept no grad alive
        torch.cuda.synchronize()
    for a, b in zip(m_a.parameters(), m_b.parameters()):
        assert torch.equal(a, b)
    if cuda_graph:
        assert o_a._cuda_graph is not None  # in-place grads: captured and replayed


def test_last_step_stats():
    """_last_step_stats after an eager step: the NS launches (one per chunk),
    the tiles they took (total_B = every bucket's B_total), the mean batch and
    the eager NS time; zeros after a graph replay (himuon.py:812-825,
    1103-1108)."""
    model = make_model(MULTI)
    opt = HiMuon(muon_groups(model), tile_size=256, b_hw=7, cuda_graph=True, cuda_graph_warmup=1)
    seed_grads(model, 31)
    opt.step()
    st = opt._last_step_stats
    plan = opt.xlayer_plan()
    n_full = sum(1 for g in opt._groups if g["full"])
    tiles_full = sum(g["tiles"].n_tiles for g in opt._groups if g["full"])
    assert st["ns_launches"] == sum(b["n_calls"] for b in plan) + n_full
    assert st["total_B"] == sum(b["B_total"] for b in plan) + tiles_full
    assert st["avg_batch"] == pytest.approx(st["total_B"] / st["ns_launches"])
    assert st["ns_gpu_ms"] > 0.0
    for k in range(3):  # capture, then replays
        seed_grads(model, 32 + k)
        opt.step()
    assert opt._cuda_graph is not None
    assert opt._last_step_stats == {"ns_gpu_ms": 0.0, "ns_launches": 0, "total_B": 0, "avg_batch": 0.0}


def test_lds_step_buckets_register_no_concat_buffer():
    """A 128 x 128-tile bucket runs its whole step in LDS (himuon_lds_step):
    it has no tile buffer, so _concat_buffers holds no entry for it; a 256
    bucket of the same model holds its bf16 (n_tiles, 256, 256) buffer."""
    model = make_model([(512, 1024), (256, 512)], torch.float32)
    groups = [{"params": [model[0].weight], "use_muon": True, "tile_size": (128, 128)},
              {"params": [model[1].weight], "use_muon": True, "tile_size": (256, 256)}]
    opt = HiMuon(groups, cuda_graph=False)
    seed_grads(model, 41)
    opt.step()
    keys = {b["bucket_key"] for b in opt.xlayer_plan()}
    assert (128, 128, False, torch.float32) in keys and (256, 256, False, torch.float32) in keys
    assert set(opt._concat_buffers) == {(256, 256, False, torch.float32)}
    buf = opt._concat_buffers[(256, 256, False, torch.float32)]
    assert buf.dtype == torch.bfloat16 and tuple(buf.shape) == (2, 256, 256)
    assert any(g["tiles"].lds_step_ok() for g in opt._groups)
