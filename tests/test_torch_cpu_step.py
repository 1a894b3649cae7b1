"""The torch-CPU restatement of the reference step (oracle/torch_cpu_step.py,
bench.py's CPU baseline) against the numpy oracle: momentum, tiling,
untiling and WD/LR exact; NS within bf16 rounding per tile (the CPU GEMM
library sums in its own order)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import himuon_oracle as O
from oracle import torch_cpu_step as T


def _rel(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


def test_momentum_and_tiling_are_exact():
    rng = np.random.default_rng(0)
    g = (rng.standard_normal((300, 700)) * 1e-3).astype(np.float32)
    buf = (rng.standard_normal((300, 700)) * 1e-3).astype(np.float32)
    e_ref, b_ref = O.momentum(g, buf, 0.95, True)
    bt = torch.from_numpy(buf.copy())
    e = T.momentum_(torch.from_numpy(g), bt, 0.95, True)
    assert np.array_equal(bt.numpy(), b_ref)
    assert np.array_equal(e.numpy(), e_ref)
    for th, tw in [(128, 256), (256, 128), (512, 512)]:
        t = T.tiles(torch.from_numpy(g), th, tw)
        ref = np.stack([O.ns_operand(x) for x in O.tile(g, th, tw)])
        assert np.array_equal(t.numpy(), ref)
        assert np.array_equal(T.untile(t, 300, 700, th, tw).numpy(), g)


@pytest.mark.parametrize("shape", [(4, 256, 256), (3, 128, 384), (256, 512), (384, 128)])
def test_newton_schulz_within_bf16_of_the_staged_oracle(shape):
    """One iteration agrees to the summation-order level (a dropped term, a
    wrong coefficient or rounding point would show as >= 1e-3); five
    iterations amplify those single bf16 roundings, as between the numpy
    oracle and the GPU kernels, and stay within 2.5e-2 per tile."""
    rng = np.random.default_rng(1)
    G = (rng.standard_normal(shape) * 1e-3).astype(np.float32)
    for steps, tol in ((1, 1e-4), (5, 2.5e-2)):
        got = T.newton_schulz(torch.from_numpy(G), steps).float().numpy()
        ref = O.ns5_staged(G, steps, round_once=len(shape) == 2)
        flat = got.reshape(-1, *got.shape[-2:]), ref.reshape(-1, *ref.shape[-2:])
        errs = [_rel(a, b) for a, b in zip(*flat)]
        assert max(errs) <= tol, (steps, errs)


def test_step_param_matches_the_oracle_step():
    rng = np.random.default_rng(2)
    h, w, tile = 700, 300, 256
    g = (rng.standard_normal((h, w)) * 1e-3).astype(np.float32)
    p0 = (rng.standard_normal((h, w)) * 0.02).astype(np.float32)
    lr, wd = 1e-2, 0.1
    pt = torch.from_numpy(p0.copy()).to(torch.bfloat16)
    bt = torch.zeros(h, w)
    upd = T.step_param(pt, torch.from_numpy(g), bt, lr, wd, tile)
    op = O.OracleParam(p=O.round_to(p0, "bfloat16"), g=g, buf=None, mu=0.95, nesterov=True, tile=(tile, tile),
                       lr=lr, wd=wd, p_dtype="bfloat16", g_dtype="float32", ns_steps=5, lr_adjust="tile")
    newp, nb, upd_ref = O.step_param(op)
    assert np.array_equal(bt.numpy(), nb)
    assert _rel(upd.numpy(), upd_ref) <= 1e-2
    # the parameter moved by the same update: compare the moves
    assert _rel(pt.float().numpy() - O.round_to(p0, "bfloat16"), newp - O.round_to(p0, "bfloat16")) <= 2e-2
