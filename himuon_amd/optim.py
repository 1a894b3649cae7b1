"""Optimizer factory: the reference's ``himuon.optim`` for ``--optimizer himuon``.

``get_optimizer("himuon", model, args)`` builds the same three param groups as
the reference (src/himuon/optim.py:116-151): Muon for 2-D weights other than
``embed_tokens``/``lm_head``; AdamW (no decay) for 1-D params; AdamW with decay
for the ``embed_tokens``/``lm_head`` matrices. ``get_optimizer_kwargs`` keeps
only non-None keys that are constructor parameters (optim.py:192-197).
The reference's other optimizers (AdamW, SOAP, Muon, MuonFsdp, HiMuonLegacy)
are outside this build and raise ``ValueError``.
"""

from __future__ import annotations

import inspect
from typing import Any, Optional, Type

from torch.optim import Optimizer

from .optimizers import HiMuon


def _himuon_groups(model: Any, optim_kwargs: dict) -> list[dict]:
    named = {name: p for name, p in model.named_parameters() if p.requires_grad}

    def is_embed_or_head(name: str) -> bool:
        return "embed_tokens" in name or "lm_head" in name

    muon = [p for n, p in named.items() if p.ndim >= 2 and not is_embed_or_head(n)]
    adamw_1d = [p for n, p in named.items() if p.ndim < 2]
    adamw_2d = [p for n, p in named.items() if p.ndim >= 2 and is_embed_or_head(n)]
    wd = optim_kwargs.get("weight_decay", 0.1)
    adamw_lr = optim_kwargs.get("adamw_lr", 1e-3)
    return [
        {"params": muon, "weight_decay": wd, "use_muon": True},
        {"params": adamw_1d, "lr": adamw_lr, "weight_decay": 0.0, "use_muon": False},
        {"params": adamw_2d, "lr": adamw_lr, "weight_decay": wd, "use_muon": False},
    ]


def get_optimizer(optimizer_name: str, model: Any, kwargs: Optional[dict | Any] = None) -> Optimizer:
    name = optimizer_name.lower()
    if name == "himuon":
        optim_kwargs = get_optimizer_kwargs(HiMuon, kwargs)
        return HiMuon(_himuon_groups(model, optim_kwargs), **optim_kwargs)
    raise ValueError(f"Optimizer {optimizer_name} not supported")


def get_optimizer_kwargs(optimizer_class: Type[Optimizer], kwargs: Optional[dict | Any] = None) -> dict:
    if kwargs is None:
        kwargs = {}
    elif not isinstance(kwargs, dict):
        kwargs = vars(kwargs)
    keys = inspect.signature(optimizer_class).parameters.keys()
    return {k: v for k, v in kwargs.items() if k in keys and v is not None}
