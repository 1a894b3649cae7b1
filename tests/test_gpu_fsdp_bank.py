"""FSDP per-bank path (himuon.py:894-964) on world-size-1 DTensor banks.

A bank parameter is a DTensor whose rank-local shard is (N, H, W), N
matrices of one shape (fsdp_bank/qwen3_scheme.py:31-78 builds them from a
model's projections). On one rank the shard is the whole bank; the step
touches only the local shard, so no collective runs (the process group
exists only because DTensor needs a device mesh).

* tiled banks (tile smaller than a matrix): every matrix tiled and padded on
  its own, so the bank path must leave each matrix exactly where the
  non-bank path leaves the same matrix given as a plain 2-D parameter:
  parameters and momentum buffers compared bit for bit after 3 eager steps,
  the capture and a replay;
* whole-matrix banks (tile covers a matrix): NS on (N, H, W) directly, the
  batched form, block (H, W): one eager step against torch's same-dtype NS5
  and the oracle's WD/LR (himuon.py:912-918, 952-963);
* the reference's errors for a 2-D local shard and for mixed DTensor and
  plain muon parameters; xlayer_plan() stays empty and the stats count one
  NS launch per bank (himuon.py:994-1019).
"""

from __future__ import annotations

import socket

import numpy as np
import pytest
import torch

from oracle import himuon_oracle as O

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    import torch.distributed as dist
    from torch.distributed.device_mesh import init_device_mesh
    from torch.distributed.tensor import Shard, distribute_tensor

    from himuon_amd.optimizers.himuon import HiMuon

    from gpu_ref import ns5_torch_staged

LR, WD, MU = 1e-2, 0.1, 0.95


@pytest.fixture(scope="module")
def mesh():
    created = False
    torch.cuda.set_device(0)
    if not dist.is_initialized():
        with socket.socket() as s:
            s.bind(("127.0.0.1", 0))
            port = s.getsockname()[1]
        dist.init_process_group("nccl", init_method=f"tcp://127.0.0.1:{port}", rank=0, world_size=1,
                                device_id=torch.device("cuda", 0))
        created = True
    yield init_device_mesh("cuda", (1,))
    if created:
        dist.destroy_process_group()


def _bank(mesh, n, h, w, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    full = (torch.randn(n, h, w, device="cuda", generator=g) * 0.02).to(dtype)
    grad = torch.randn(n, h, w, device="cuda", generator=g) * 1e-3
    p = torch.nn.Parameter(distribute_tensor(full.clone(), mesh, [Shard(0)]))
    p.grad_dtype = torch.float32  # fp32 grads on bf16 parameters, as the configs train
    p.grad = distribute_tensor(grad.clone(), mesh, [Shard(0)])
    return p, full, grad


def test_tiled_banks_match_the_plain_parameter_path(mesh):
    specs = [(4, 1024, 512, 11), (6, 256, 768, 12), (3, 700, 300, 13)]  # the last pads per matrix
    banks, plain = [], []
    for n, h, w, seed in specs:
        p, full, grad = _bank(mesh, n, h, w, torch.bfloat16, seed)
        banks.append(p)
        for i in range(n):
            q = torch.nn.Parameter(full[i].clone())
            q.grad_dtype = torch.float32
            q.grad = grad[i].clone()
            plain.append(q)
    print(f"[fsdp bank] tiled: {[s[:3] for s in specs]}", flush=True)
    ob = HiMuon([{"params": banks, "use_muon": True}], lr=LR, weight_decay=WD, tile_size=256)
    op = HiMuon([{"params": plain, "use_muon": True}], lr=LR, weight_decay=WD, tile_size=256)
    for k in range(5):  # 3 eager steps, capture (+ its replay), one replay
        ob.step()
        op.step()
        if k == 0:
            assert ob._last_step_stats["ns_launches"] == len(banks)
    torch.cuda.synchronize()
    assert ob._cuda_graph is not None and ob.xlayer_plan() == []
    j = 0
    for p, (n, h, w, _) in zip(banks, specs):
        local, buf = p.to_local(), ob.state[p]["momentum_buffer"]
        assert buf.shape == (n, h, w)
        for i in range(n):
            q = plain[j]
            assert torch.equal(local[i], q.data), f"bank {n}x{h}x{w} matrix {i}: parameters differ"
            assert torch.equal(buf[i], op.state[q]["momentum_buffer"]), f"bank matrix {i}: momentum differs"
            j += 1


@pytest.mark.parametrize("h,w", [(256, 384), (384, 256)])
def test_whole_matrix_bank_runs_batched_ns_with_block_hw(mesh, h, w):
    n = 5
    print(f"[fsdp bank] whole-matrix {n}x{h}x{w}", flush=True)
    p, full, grad = _bank(mesh, n, h, w, torch.bfloat16, 21)
    opt = HiMuon([{"params": [p], "use_muon": True}], lr=LR, weight_decay=WD, tile_size=512, cuda_graph=False)
    opt.step()
    torch.cuda.synchronize()
    g = grad.cpu().numpy()
    e, buf = O.momentum(g, np.zeros_like(g), MU, True)
    assert np.array_equal(opt.state[p]["momentum_buffer"].cpu().numpy(), buf)
    # NS on (N, H, W): the batched form (B X rounded before + a X)
    X = ns5_torch_staged(torch.from_numpy(e).cuda(), round_once=False).float().cpu().numpy()
    scale = np.float32(opt.adjust_lr_for_muon(1.0, (h, w)))
    upd = O.round_to(O.round_to(X, "float32") * scale, "float32")
    exp = O.apply_update(full.float().cpu().numpy(), upd, LR, WD, "bfloat16", "float32")
    assert np.array_equal(p.to_local().detach().float().cpu().numpy(), exp)


def test_bank_path_errors(mesh):
    p2, _, _ = _bank(mesh, 1, 256, 256, torch.bfloat16, 31)
    flat = torch.nn.Parameter(distribute_tensor(p2.to_local()[0].detach().clone(), mesh, [Shard(0)]))
    flat.grad_dtype = torch.float32
    flat.grad = distribute_tensor(torch.zeros(256, 256, device="cuda"), mesh, [Shard(0)])
    with pytest.raises(RuntimeError, match="requires bank-wrapped 3D"):
        HiMuon([{"params": [flat], "use_muon": True}], tile_size=128, cuda_graph=False).step()
    q = torch.nn.Parameter(torch.zeros(256, 256, device="cuda", dtype=torch.bfloat16))
    q.grad_dtype = torch.float32
    q.grad = torch.zeros(256, 256, device="cuda")
    with pytest.raises(RuntimeError, match="non-DTensor param"):
        HiMuon([{"params": [p2, q], "use_muon": True}], tile_size=128, cuda_graph=False).step()
