"""himuon_ns5_noalloc (no workspace argument: the A/B intermediates live in
the library's own device array) against himuon_ns5_ex with a caller
workspace, both through the C ABI: bit-identical outputs on calls in a row,
the second with a smaller input, so the second runs on a scratch array that
still holds the first call's contents.

* call 1: 160 tiles of 512 x 512, 5 steps (the 64 MiB array holds 64 tiles'
  A and B: sub-batches of 64, 64 and 32);
* call 2: 7 tiles of 512 x 512, 5 steps;
* call 3: 3 tiles of 256 x 1024 with the 2-D rounding flag, 2 steps.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

if torch.cuda.is_available():
    from himuon_amd import _native as nat

DEV = "cuda"


def _tiles(n, mp, np_, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, mp, np_, generator=g) * 1e-3).to(torch.bfloat16).to(DEV)
    inv = (1.0 / x.float().flatten(1).norm(dim=1)).contiguous()
    return x, inv


def _with_workspace(x, inv, n, mp, np_, steps, flags):
    xr, yr = x.clone(), torch.full_like(x, float("nan"))
    sb = nat.default_sub_batch(n, mp, np_)
    ws = torch.empty(nat.ns5_workspace_bytes(sb, mp, np_), device=DEV, dtype=torch.uint8)
    rc = nat.load().himuon_ns5_ex(xr.data_ptr(), yr.data_ptr(), inv.data_ptr(), n, mp, np_, steps, nat.NS_A,
                                  nat.NS_B, nat.NS_C, ws.data_ptr(), ws.numel(), sb, flags, nat._stream())
    assert rc == 0, nat.load().himuon_error_string(rc)
    torch.cuda.synchronize()
    return xr if steps % 2 == 0 else yr


def _no_alloc(x, inv, n, mp, np_, steps, flags):
    xn, yn = x.clone(), torch.full_like(x, float("nan"))
    rc = nat.load().himuon_ns5_noalloc(xn.data_ptr(), yn.data_ptr(), inv.data_ptr(), n, mp, np_, steps, nat.NS_A,
                                       nat.NS_B, nat.NS_C, flags, nat._stream())
    assert rc == 0, nat.load().himuon_error_string(rc)
    torch.cuda.synchronize()
    return xn if steps % 2 == 0 else yn


def test_ns5_noalloc_matches_the_workspace_entry_point():
    calls = [(160, 512, 512, 5, 0, 1), (7, 512, 512, 5, 0, 2), (3, 256, 1024, 2, nat.NS_ROUND_ONCE, 3)]
    for n, mp, np_, steps, flags, seed in calls:
        print(f"[ns5_noalloc] {n} x {mp}x{np_} steps={steps} flags={flags:#x}", flush=True)
        x, inv = _tiles(n, mp, np_, seed)
        ref = _with_workspace(x, inv, n, mp, np_, steps, flags)
        got = _no_alloc(x, inv, n, mp, np_, steps, flags)
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got, ref), f"{n} x {mp}x{np_}: max |d| {(got.float() - ref.float()).abs().max().item()}"


def test_ns5_noalloc_rejects_a_tile_larger_than_its_array():
    # mp = np = 4224: one tile's A and B (4 mp^2 bytes) exceed 64 MiB
    rc = nat.load().himuon_ns5_noalloc(8, 16, 24, 1, 4224, 4224, 5, 1.0, 1.0, 1.0, 0, None)
    assert rc == -28
