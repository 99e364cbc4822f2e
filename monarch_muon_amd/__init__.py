"""MI355X-native Monarch-Muon optimizer step (gfx950 HIP kernels behind a C ABI).

Drop-in for the reference's ``MonarchMuonOptimizer`` (``--opt monarch_muon``)
and its FP8-state variant ``CoatStateMonarchMuon``.
"""
from .optim import CoatStateMonarchMuon, MonarchMuonOptimizer, QuantizationConfig

__all__ = ["MonarchMuonOptimizer", "CoatStateMonarchMuon", "QuantizationConfig"]
