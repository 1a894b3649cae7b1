"""himuon_amd — the HiMuon optimizer step as MI355X-native HIP kernels.

Drop-in for the reference's ``himuon.optim.get_optimizer("himuon", ...)`` and
``himuon.optimizers.HiMuon``; see ``himuon_amd.optim`` and
``himuon_amd.optimizers.himuon``.
"""

from .optimizers import HiMuon

__all__ = ("HiMuon",)
__version__ = "0.1.0"
