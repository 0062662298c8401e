"""ElasticBit adaptive threshold-driven weight compression (MI355X / gfx950)."""

from .core import BackendInfo, BitAnalysis, BitCandidate, ElasticBit, RuntimeMatrix

__all__ = ["ElasticBit", "RuntimeMatrix", "BitAnalysis", "BitCandidate", "BackendInfo"]
