"""CPU contract of the optimizer factory (reference: src/himuon/optim.py:116-151,
192-197; tests/unit/test_optimizer_factory.py)."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn

from himuon_amd.optim import get_optimizer, get_optimizer_kwargs
from himuon_amd.optimizers.himuon import HiMuon


class TinyLM(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed_tokens = nn.Embedding(32, 16)
        self.norm = nn.LayerNorm(16)
        self.mlp = nn.Linear(16, 24)
        self.lm_head = nn.Linear(16, 32, bias=False)


@pytest.fixture
def m():
    torch.manual_seed(0)
    return TinyLM()


def ids(ps):
    return {id(p) for p in ps}


def test_three_groups(m):
    opt = get_optimizer("himuon", m, SimpleNamespace())
    assert isinstance(opt, HiMuon) and len(opt.param_groups) == 3


def test_routing(m):
    opt = get_optimizer("HiMuon", m, SimpleNamespace())
    muon = [g for g in opt.param_groups if g["use_muon"]]
    adamw = [g for g in opt.param_groups if not g["use_muon"]]
    assert len(muon) == 1 and ids(muon[0]["params"]) == {id(m.mlp.weight)}
    nodecay = [g for g in adamw if g["weight_decay"] == 0.0]
    decay = [g for g in adamw if g["weight_decay"] != 0.0]
    assert ids(nodecay[0]["params"]) == {id(m.norm.weight), id(m.norm.bias), id(m.mlp.bias)}
    assert ids(decay[0]["params"]) == {id(m.embed_tokens.weight), id(m.lm_head.weight)}
    assert all(g["lr"] == 1e-3 for g in adamw)


def test_partition_complete_and_disjoint(m):
    opt = get_optimizer("himuon", m, SimpleNamespace())
    grouped = [id(p) for g in opt.param_groups for p in g["params"]]
    assert len(grouped) == len(set(grouped))
    assert set(grouped) == ids(p for p in m.parameters() if p.requires_grad)


def test_cli_kwargs_reach_constructor(m):
    args = SimpleNamespace(lr=0.01, weight_decay=0.2, tile_size=256, cuda_graph=False, adamw_lr=5e-4, batch_size=8)
    opt = get_optimizer("himuon", m, args)
    g = opt.param_groups[0]
    assert g["lr"] == 0.01 and g["weight_decay"] == 0.2 and g["tile_size"] == (256, 256)
    assert opt._cuda_graph_enabled is False
    # adamw_lr is not a constructor parameter: filtered out, default 1e-3 used
    assert opt.param_groups[1]["lr"] == 1e-3


def test_kwarg_filtering():
    ns = SimpleNamespace(lr=0.01, weight_decay=0.2, not_a_param=5, momentum=None)
    assert get_optimizer_kwargs(HiMuon, ns) == {"lr": 0.01, "weight_decay": 0.2}
    assert get_optimizer_kwargs(HiMuon, None) == {}


def test_unknown_name(m):
    with pytest.raises(ValueError):
        get_optimizer("not-an-optimizer", m, SimpleNamespace())
