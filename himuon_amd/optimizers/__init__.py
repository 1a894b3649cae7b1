"""Optimizers of the MI355X HiMuon path (the reference's ``himuon.optimizers``)."""

from .himuon import HiMuon

__all__ = ("HiMuon",)
