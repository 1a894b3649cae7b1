"""CPU contract of the HiMuon public surface (no step() — that needs the GPU).

Same contract as the reference's tests/unit/test_optimizer_api.py: constructor
signature and defaults, param-group schema, tile_size normalisation,
reconfigure semantics, state_dict round trip, and the calls the training
script makes around step() (scheduler, zero_grad modes, reconfigure).
"""

from __future__ import annotations

import inspect
import warnings
from types import SimpleNamespace

import pytest
import torch
import torch.nn as nn
from torch.optim import Optimizer

from himuon_amd.optim import get_optimizer
from himuon_amd.optimizers.himuon import HiMuon

# Constructor defaults of the reference (himuon.py:64-80).
REFERENCE_DEFAULTS = {
    "lr": 0.02,
    "momentum": 0.95,
    "nesterov": True,
    "weight_decay": 0.1,
    "tile_size": 512,
    "ns_steps": 5,
    "use_muon": True,
    "lr_adjust": "tile",
    "adamw_betas": (0.95, 0.95),
    "adamw_eps": 1e-8,
    "b_hw": None,
    "cuda_graph": True,
    "cuda_graph_warmup": 3,
}

GROUP_KEYS = {"lr", "momentum", "nesterov", "weight_decay", "tile_size", "ns_steps", "use_muon",
              "adamw_betas", "adamw_eps"}


class TinyLM(nn.Module):
    """Module names the factory routes on: embed_tokens / lm_head -> AdamW 2-D,
    the inner Linear weight -> Muon, 1-D params -> AdamW no-decay."""

    def __init__(self):
        super().__init__()
        self.embed_tokens = nn.Embedding(32, 16)
        self.norm = nn.LayerNorm(16)
        self.mlp = nn.Linear(16, 24)
        self.lm_head = nn.Linear(16, 32, bias=False)


@pytest.fixture
def tiny_lm():
    torch.manual_seed(0)
    return TinyLM()


def _one(p):
    return [{"params": [p], "use_muon": True}]


def test_signature_matches_reference():
    params = {k: v for k, v in inspect.signature(HiMuon.__init__).parameters.items() if k not in ("self", "params")}
    assert set(params) == set(REFERENCE_DEFAULTS)
    for k, v in REFERENCE_DEFAULTS.items():
        assert params[k].default == v, k


def test_is_optimizer_with_group_keys():
    opt = HiMuon(_one(nn.Parameter(torch.zeros(8, 8))))
    assert isinstance(opt, Optimizer)
    for g in opt.param_groups:
        assert GROUP_KEYS <= set(g)


@pytest.mark.parametrize("given,expected", [(512, (512, 512)), ((128, 256), (128, 256)), ([64, 32], (64, 32))])
def test_tile_size_normalised(given, expected):
    opt = HiMuon(_one(nn.Parameter(torch.zeros(8, 8))), tile_size=given)
    assert all(g["tile_size"] == expected for g in opt.param_groups)


@pytest.mark.parametrize("bad", [(512, 0), (0, 0), (-1, 4)])
def test_tile_size_must_be_positive(bad):
    with pytest.raises(AssertionError):
        HiMuon(_one(nn.Parameter(torch.zeros(8, 8))), tile_size=bad)


def test_lr_adjust_validated():
    with pytest.raises(ValueError):
        HiMuon(_one(nn.Parameter(torch.zeros(8, 8))), lr_adjust="spectral")


def test_adjust_lr_for_muon():
    opt = HiMuon(_one(nn.Parameter(torch.zeros(8, 8))))
    assert opt.adjust_lr_for_muon(1e-2, (256, 256)) == pytest.approx(0.032)
    assert opt.adjust_lr_for_muon(1.0, (1024, 3072)) == pytest.approx(0.2 * 3072**0.5)
    opt.lr_adjust = "none"
    assert opt.adjust_lr_for_muon(1e-2, (256, 256)) == 1e-2


class TestReconfigure:
    def test_writes_all_groups_and_normalises(self):
        a, b = nn.Parameter(torch.zeros(16, 16)), nn.Parameter(torch.zeros(8))
        opt = HiMuon([
            {"params": [a], "use_muon": True, "tile_size": (128, 128)},
            {"params": [b], "use_muon": False, "tile_size": (128, 128)},
        ])
        opt.reconfigure(tile_size=256, lr=0.05, weight_decay=0.3)
        for g in opt.param_groups:
            assert (g["tile_size"], g["lr"], g["weight_decay"]) == ((256, 256), 0.05, 0.3)

    def test_tuple_kept_and_unknown_ignored(self):
        opt = HiMuon(_one(nn.Parameter(torch.zeros(16, 16))))
        opt.reconfigure(tile_size=(128, 256), not_a_key=1)
        g = opt.param_groups[0]
        assert g["tile_size"] == (128, 256) and "not_a_key" not in g

    def test_clears_cached_state(self):
        opt = HiMuon(_one(nn.Parameter(torch.zeros(16, 16))))
        opt._cached_plan = [{"x": 1}]
        opt._concat_buffers[("k",)] = torch.zeros(1)
        opt._pending_updates.append(("p", "u", 0))
        opt._graph_step_count = 5
        opt.reconfigure(tile_size=64)
        assert opt._cached_plan is None and opt._concat_buffers == {} and opt._pending_updates == []
        assert opt._graph_step_count == 0 and opt._cuda_graph is None and opt.xlayer_plan() == []


def test_state_dict_round_trip():
    opt = HiMuon(_one(nn.Parameter(torch.zeros(8, 8))))
    sd = opt.state_dict()
    assert {"state", "param_groups"} <= set(sd)
    opt2 = HiMuon(_one(nn.Parameter(torch.zeros(8, 8))))
    opt2.load_state_dict(sd)
    assert len(opt2.param_groups) == 1


def test_step_without_gpu_raises():
    """No CPU implementation: step() on CPU tensors fails loudly."""
    p = nn.Parameter(torch.zeros(8, 8))
    p.grad = torch.ones(8, 8)
    opt = HiMuon(_one(p), cuda_graph=False)
    with pytest.raises(RuntimeError):
        opt.step()


def test_balanced_chunks_matches_reference_formula():
    assert HiMuon._balanced_chunks(13860, 11059) == [6930, 6930]
    assert HiMuon._balanced_chunks(10, 3) == [3, 3, 2, 2]
    assert HiMuon._balanced_chunks(0, 3) == []


def test_tile_untile_helpers_round_trip():
    x = torch.randn(70, 45)
    t, info = HiMuon._tile(x, (32, 16))
    assert t.shape == (3, 3, 32, 16)
    assert torch.equal(HiMuon._untile(t, info), x)


class TestTrainLoopSurface:
    """Calls train.py makes around step() (scheduler, zero_grad, reconfigure)."""

    def _opt(self, model):
        return get_optimizer("himuon", model, SimpleNamespace())

    def test_numeric_lr_in_every_group(self, tiny_lm):
        assert all(isinstance(g["lr"], (int, float)) for g in self._opt(tiny_lm).param_groups)

    def test_cosine_schedule_drives_lr(self, tiny_lm):
        from transformers import get_cosine_schedule_with_warmup

        opt = self._opt(tiny_lm)
        base = opt.param_groups[0]["lr"]
        sched = get_cosine_schedule_with_warmup(opt, num_warmup_steps=3, num_training_steps=12)
        lrs = [opt.param_groups[0]["lr"]]
        with warnings.catch_warnings():
            warnings.filterwarnings("ignore", message="Detected call of")
            for _ in range(12):
                sched.step()
                lrs.append(opt.param_groups[0]["lr"])
        assert lrs[0] == pytest.approx(0.0, abs=1e-12)
        assert lrs[3] == pytest.approx(base)
        assert lrs[-1] < lrs[3]

    def test_zero_grad_modes(self, tiny_lm):
        opt = self._opt(tiny_lm)
        ps = [p for g in opt.param_groups for p in g["params"]]
        for p in ps:
            p.grad = torch.ones_like(p)
        opt.zero_grad(set_to_none=False)
        assert all(p.grad is not None and not p.grad.any() for p in ps)
        opt.zero_grad(set_to_none=True)
        assert all(p.grad is None for p in ps)

    def test_reconfigure_surface(self, tiny_lm):
        opt = self._opt(tiny_lm)
        assert hasattr(opt, "reconfigure")
        opt.reconfigure(tile_size=256, lr=0.05)
        assert opt.param_groups[0]["tile_size"] == (256, 256) and opt.param_groups[0]["lr"] == 0.05
