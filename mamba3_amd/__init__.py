"""MI355X-native Mamba-3 mixer hot path (drop-in for jreoka/mamba3's ``Mamba3``)."""

from .model import Mamba3

__all__ = ["Mamba3"]
