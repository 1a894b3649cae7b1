"""Parity at every benchmark workload (cfg2-cfg5) on the GPU.

Each test builds a config's full parameter set exactly as bench.py does
(seeded device generator: bf16 or fp32 params, fp32 grads ~N(0, 1e-3^2)),
runs HiMuon.step() through the reference's state machine (3 eager warm-up
steps, capture with its first replay, one more replay; himuon.py:1074-1109),
and checks, with the grads copied to the host where the oracle needs them:

* momentum buffers of whole sampled matrices bit-exact against
  oracle.momentum applied once per step (the grads stay in place, as a
  training loop with zero_grad(set_to_none=False) keeps them);
* tiles sampled across every sub-batch, including tiles whose offset in the
  tile buffer is past 4 GiB: where the bucket stores its NS result (cfg3's
  full-matrix groups), the NS tiles against the reference's NS5 in the same
  dtypes (torch on the GPU, ns5_torch_staged): the north star's per-tile
  relative Frobenius error <= 1e-2 and bit-identical as built, their singular
  values against the quintic's band, every NS output finite;
* the parameters of the sampled tiles after the last replay bit-exact against
  oracle.apply_update of the sampled NS tile, or of torch's NS5 of the same
  inputs where no NS result is stored (WD/LR fused in the untile).

cfg5's 128 x 128-tile bucket runs the whole step in LDS (himuon_lds_step), and
the 512 x 512-tile buckets (cfg2, cfg4, cfg5 after reconfigure) apply the untile
with WD/LR inside the last NS iteration (himuon_ns5_untile_apply): neither stores
an NS result, so their check is the parameters of the sampled tiles against
oracle.apply_update of torch's NS5 of the same inputs (tests/test_gpu_lds_step.py
and tests/test_gpu_ns_untile.py pin those kernels bit for bit against the
separate launches, whose NS tiles tests/test_gpu_kernels.py checks).

Full-matrix groups (cfg3) compare against the 2-D third product of the
reference (torch.addmm, himuon.py:249-253). cfg5 runs the tile-128 regime,
then reconfigure(tile_size=512) and the same sequence again (recapture).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import bench
from oracle import himuon_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from himuon_amd.optimizers.himuon import HiMuon

    from gpu_ref import ns5_torch_staged, per_tile_rel_fro

LR, WD, MU = 1e-2, 0.1, 0.95
N_STEPS = 5  # 3 eager warm-up steps, capture (+ its replay), one replay


def _build(config):
    layers, shapes, tile, pdtype, _ = bench.CONFIGS[config]
    params = bench.build_params(layers, shapes, pdtype, seed=0)
    opt = HiMuon([{"params": params, "use_muon": True}], lr=LR, weight_decay=WD, tile_size=tile,
                 cuda_graph=True, cuda_graph_warmup=3)
    return params, opt


def _locate(grp, t):
    """(param index, tile row, tile column) of bucket tile t."""
    i = int(np.searchsorted(np.asarray(grp.tile0), t, side="right")) - 1
    r, c = divmod(t - grp.tile0[i], -(-grp.params[i].shape[1] // grp.tile_w))
    return i, r, c


def _region(x, r, c, th, tw):
    h, w = x.shape
    out = torch.zeros((th, tw), dtype=x.dtype, device=x.device)
    rr, cc = min(th, h - r * th), min(tw, w - c * tw)
    out[:rr, :cc] = x[r * th : r * th + rr, c * tw : c * tw + cc]
    return out, rr, cc


def _momentum_steps(g, n, mu=MU):
    """oracle.momentum n times from a zero buffer with the same grad; returns
    (NS input of the last step, buffer after it)."""
    buf = np.zeros_like(g)
    for _ in range(n):
        e, buf = O.momentum(g, buf, mu, True)
    return e, buf


def _check_group(opt, gi, sample, n_steps, p_before, round_once=False, label=""):
    """Sampled tiles of group gi after n_steps steps: NS output vs torch's
    same-dtype NS5, momentum region bit-exact, band, fused-untile parameters."""
    g = opt._groups[gi]
    grp = g["tiles"]
    # 128 x 128-tile buckets run the whole step in LDS (himuon_lds_step), and
    # 512 x 512-tile buckets apply the untile inside the last NS iteration
    # (himuon_ns5_untile_apply): no NS result is stored, the parameters are
    # the output checked
    no_tiles = (opt._fuse_lds_step and grp.lds_step_ok()) or (opt._fuse_ns_untile and grp.ns_untile_ok(g["steps"]))
    res = None if no_tiles else grp.result(g["steps"])
    if not no_tiles:
        assert torch.isfinite(res.float()).all(), f"{label}: non-finite NS output"
    th, tw, m, n = grp.tile_h, grp.tile_w, grp.m, grp.n
    inputs, outs = [], []
    for t in sample:
        i, r, c = _locate(grp, t)
        p = grp.params[i]
        gt, rr, cc = _region(p.grad, r, c, th, tw)
        e, buf = _momentum_steps(gt.cpu().numpy(), n_steps)
        mb = opt.state[p]["momentum_buffer"][r * th : r * th + rr, c * tw : c * tw + cc]
        assert np.array_equal(mb.cpu().numpy(), buf[:rr, :cc]), f"{label}: momentum tile {t} not bit-exact"
        inputs.append(torch.from_numpy(e))
        if res is not None:
            out = res[t, :m, :n]
            outs.append(out.transpose(0, 1) if grp.trans else out)
    X = torch.stack(inputs).to("cuda")
    ref = ns5_torch_staged(X, steps=g["steps"], round_once=round_once)
    if no_tiles:
        print(f"  {label}: NS result not stored: {len(sample)} tiles' parameters vs torch NS5 + oracle WD/LR",
              flush=True)
        assert torch.isfinite(ref).all()
        _check_params(grp, sample, ref.float(), p_before, label)
        return
    got = torch.stack(outs).float()
    err = per_tile_rel_fro(got, ref.float())
    print(f"  {label}: {len(sample)} tiles vs torch NS5: max {err.max():.2e} "
          f"(bit-identical: {torch.equal(got, ref.float())})", flush=True)
    assert err.max() <= 1e-2, err
    assert torch.equal(got, ref.float()), f"{label}: NS tiles differ from torch's same-dtype NS5"
    # singular values: inside the quintic band of each tile's normalised spectrum
    for k in range(min(8, len(sample))):
        sv = torch.linalg.svdvals(got[k].double()).cpu().numpy()
        sin = torch.linalg.svdvals(X[k].double()).cpu().numpy()
        sin = sin / np.linalg.norm(sin)
        floor = 4e-3
        lo, hi = O.quintic_band(max(sin.min(), floor), sin.max())
        assert sv.max() <= hi + 0.03
        assert (sv < lo - 0.03).sum() <= int((sin < floor).sum())
    _check_params(grp, sample, got, p_before, label)


def _check_params(grp, sample, x, p_before, label):
    """Parameters of the sampled tiles (WD/LR applied by the fused untile)
    bit-exact against oracle.apply_update of the NS tiles x (per sample)."""
    th, tw = grp.tile_h, grp.tile_w
    if grp.fused and p_before is not None:
        pdt = "bfloat16" if grp.params[0].dtype == torch.bfloat16 else "float32"
        scale = np.float32(grp.upd_scales[0])
        for k, t in enumerate(sample):
            i, r, c = _locate(grp, t)
            p = grp.params[i]
            u = x[k].cpu().numpy()[: min(th, p.shape[0] - r * th), : min(tw, p.shape[1] - c * tw)]
            upd = O.round_to(O.round_to(u, "float32") * scale, "float32")
            exp = O.apply_update(p_before[t], upd, LR, WD, pdt, "float32")
            now = p.data[r * th : r * th + u.shape[0], c * tw : c * tw + u.shape[1]].float().cpu().numpy()
            assert np.array_equal(now, exp), f"{label}: parameter region of tile {t} not bit-exact"


def _snapshot(grp, sample):
    out = {}
    for t in sample:
        i, r, c = _locate(grp, t)
        p = grp.params[i]
        out[t] = p.data[r * grp.tile_h : (r + 1) * grp.tile_h, c * grp.tile_w : (c + 1) * grp.tile_w].float().cpu().numpy()
    return out


def _run(opt, n):
    for k in range(n):
        opt.step()
    torch.cuda.synchronize()


def _whole_momentum(opt, params, idx, n_steps):
    for i in idx:
        p = params[i]
        _, buf = _momentum_steps(p.grad.cpu().numpy(), n_steps)
        assert np.array_equal(opt.state[p]["momentum_buffer"].cpu().numpy(), buf), f"momentum of param {i}"


def _tiled_sample(n_tiles, sub_batch, extra=()):
    """~32 tile indices spread over every sub-batch: first, last and middle
    tiles of each, plus `extra`."""
    s = set(extra)
    for b0 in range(0, n_tiles, sub_batch):
        b1 = min(n_tiles, b0 + sub_batch) - 1
        s.update({b0, b0 + 1, (b0 + b1) // 2, b1})
    rng = np.random.default_rng(0)
    s.update(int(v) for v in rng.integers(0, n_tiles, size=max(0, 32 - len(s))))
    return sorted(s)


def _tiled_config(config, whole_idx, extra=()):
    print(f"[config] {config}", flush=True)
    params, opt = _build(config)
    _run(opt, N_STEPS - 1)
    assert opt._cuda_graph is not None, "graph not captured after warm-up"
    grp = opt._groups[0]["tiles"]
    sample = _tiled_sample(grp.n_tiles, opt._groups[0]["sub_batch"], extra)
    before = _snapshot(grp, sample)
    _run(opt, 1)  # a replay
    _whole_momentum(opt, params, whole_idx, N_STEPS)
    _check_group(opt, 0, sample, N_STEPS, before, label=config)
    return params, opt


def test_cfg2_qwen3_0p6b_tile512():
    params, opt = _tiled_config("qwen3-0.6b", whole_idx=[0, 4, 6])
    assert opt._groups[0]["tiles"].n_tiles == 1680


def test_cfg4_qwen3_4b_tile512():
    """The headline config: 13,860 tiles; tiles past 8,192 sit beyond 4 GiB
    of the bf16 tile buffer; 9728x2560 and 2560x9728 matrices sampled whole."""
    params, opt = _tiled_config("qwen3-4b", whole_idx=[4, 6, 0], extra=(8192, 8193, 12000, 13859))
    grp = opt._groups[0]["tiles"]
    assert grp.n_tiles == 13860 and grp.tiles.numel() * 2 > (6 << 30)  # 7.27 GB


def test_cfg3_qwen3_0p6b_full_matrix():
    """Full-matrix mode: 7 shape groups of 28 matrices each run as batched
    NS (f3), every matrix one tile, against the reference's 2-D NS
    (torch.addmm third product) per matrix."""
    config = "qwen3-0.6b-full"
    print(f"[config] {config}", flush=True)
    params, opt = _build(config)
    _run(opt, N_STEPS - 1)
    groups = opt._groups
    assert all(g["full"] for g in groups)
    # q 2048x1024, k/v 1024x1024, o 1024x2048, gate/up 3072x1024, down 1024x3072
    assert sorted(g["tiles"].n_tiles for g in groups) == [28, 28, 28, 56, 56]
    samples = {gi: sorted({0, 1, g["tiles"].n_tiles // 2, g["tiles"].n_tiles - 1}) for gi, g in enumerate(groups)}
    before = {gi: _snapshot(groups[gi]["tiles"], s) for gi, s in samples.items()}
    _run(opt, 1)
    _whole_momentum(opt, params, [0, 4, 6], N_STEPS)
    for gi, s in samples.items():
        g = groups[gi]["tiles"]
        _check_group(opt, gi, s, N_STEPS, before[gi], round_once=True, label=f"{config} {g.tile_h}x{g.tile_w}")


def test_cfg5_llama3_8b_tile128_then_reconfigure_512():
    config = "llama3-8b-t128"
    print(f"[config] {config}", flush=True)
    params, opt = _build(config)
    _run(opt, N_STEPS - 1)
    grp = opt._groups[0]["tiles"]
    assert grp.n_tiles == 425984 and grp.mp == 128
    sample = _tiled_sample(grp.n_tiles, opt._groups[0]["sub_batch"], extra=(425983, 300000))
    before = _snapshot(grp, sample)
    _run(opt, 1)
    _whole_momentum(opt, params, [0, 4], N_STEPS)
    _check_group(opt, 0, sample, N_STEPS, before, label=f"{config} T=128")
    del before
    # mid-run reconfigure: plan, buffers and graph dropped; 3 eager steps, recapture, replay
    opt.reconfigure(tile_size=512)
    assert opt._cuda_graph is None and opt._groups is None
    _run(opt, N_STEPS - 1)
    assert opt._cuda_graph is not None
    grp = opt._groups[0]["tiles"]
    assert grp.n_tiles == 26624 and grp.mp == 512
    sample = _tiled_sample(grp.n_tiles, opt._groups[0]["sub_batch"], extra=(26623,))
    before = _snapshot(grp, sample)
    _run(opt, 1)
    _whole_momentum(opt, params, [6], 2 * N_STEPS)
    _check_group(opt, 0, sample, 2 * N_STEPS, before, label=f"{config} after reconfigure(512)")


@pytest.mark.parametrize("cuda_graph", [False, True])
def test_cfg1_single_matrix_step(cuda_graph):
    """cfg1 end to end: one 1024 x 1024 fp32 weight, fp32 grads ~N(0, 1e-3^2)
    from a seed (new values every step), Nesterov momentum 0.95, tile 256 (16
    NS tiles), lr 1e-2, wd 0.1, five steps (graph mode: two eager warm-up
    steps, the capture with its replay, two replays). After every step:
    * the momentum buffer equals oracle.momentum bit for bit;
    * the parameter equals the oracle's step from the GPU's previous parameter
      (momentum, tiling, untiling, lr scale 0.2 sqrt(256) and WD/LR roundings)
      around torch's same-dtype NS5 on the GPU, bit for bit;
    * the update of every NS tile is within the numpy oracle's NS5 noise floor
      (per-tile relative Frobenius max 2e-2, mean 1e-2);
    * the parameter is within the reference's 1e-2 self-consistency tolerance
      of the numpy oracle's own trajectory (test_himuon_self_consistency.py:18)."""
    print(f"[cfg1] cuda_graph={cuda_graph}", flush=True)
    layers, shapes, T, pdtype, _ = bench.CONFIGS["cfg1"]
    assert (layers, shapes, T, pdtype) == (1, [(1024, 1024)], 256, torch.float32)
    gen = torch.Generator().manual_seed(1)
    p = torch.nn.Parameter((torch.randn(1024, 1024, generator=gen) * 0.02).to("cuda"))
    opt = HiMuon([{"params": [p], "use_muon": True}], lr=LR, weight_decay=WD, momentum=MU, nesterov=True,
                 tile_size=T, cuda_graph=cuda_graph, cuda_graph_warmup=2)
    ts = opt.param_groups[0]["tile_size"]
    p_np = p.detach().cpu().numpy()
    buf = None

    def torch_ns(x, steps):
        return ns5_torch_staged(torch.from_numpy(x).to("cuda"), steps).float().cpu().numpy()

    for k in range(5):
        g = (torch.randn(1024, 1024, generator=gen) * 1e-3)
        if p.grad is None:
            p.grad = torch.empty_like(p)
        p.grad.copy_(g.to("cuda"))
        prev = p.detach().cpu().numpy()
        opt.step()
        torch.cuda.synchronize()
        gn = g.numpy()
        got = p.detach().cpu().numpy()
        op = O.OracleParam(p=prev, g=gn, buf=buf, tile=ts, lr=LR, wd=WD)
        exp_t, nb, _ = O.step_param(op, ns=torch_ns)
        exp_o, _, _ = O.step_param(op)
        assert np.array_equal(opt.state[p]["momentum_buffer"].cpu().numpy(), nb), k
        assert np.array_equal(got, exp_t), (k, int((got != exp_t).sum()))
        base = prev * np.float32(1 - LR * WD)
        d_got, d_exp = got - base, exp_o - base
        errs = np.array([np.linalg.norm(d_got[r:r + T, c:c + T] - d_exp[r:r + T, c:c + T])
                         / np.linalg.norm(d_exp[r:r + T, c:c + T]) for r in range(0, 1024, T) for c in range(0, 1024, T)])
        print(f"  step {k}: update vs numpy oracle per tile max {errs.max():.4f} mean {errs.mean():.4f}", flush=True)
        assert errs.max() <= 2e-2 and errs.mean() <= 1e-2
        op_o = O.OracleParam(p=p_np, g=gn, buf=buf, tile=ts, lr=LR, wd=WD)
        p_np, _, _ = O.step_param(op_o)
        np.testing.assert_allclose(got, p_np, rtol=1e-2, atol=1e-2)
        buf = nb
    if cuda_graph:
        assert opt._cuda_graph is not None
