"""``sluice.offloader``: the offloader module of the reference package
(src/sluice/offloader.py), implemented in sluice_amd.offloader."""

from sluice_amd.offloader import NON_EXPERT_WEIGHTS, ExpertStreamOffloader

__all__ = ["ExpertStreamOffloader", "NON_EXPERT_WEIGHTS"]
