"""MI355X-native Monarch-Muon optimizer step (gfx950 HIP kernels behind a C ABI).

Drop-in for the reference's ``MonarchMuonOptimizer`` (``--opt monarch_muon``)
and its FP8-state variant ``CoatStateMonarchMuon``, plus the Monarch butterfly
multiply (``butterfly_blk``) whose backward produces the gradients they consume.
"""
from .butterfly import butterfly_blk, butterfly_blk_bwd_op, butterfly_blk_op, patch_monarch_linear
from .optim import CoatStateMonarchMuon, MonarchMuonOptimizer, QuantizationConfig

__all__ = ["MonarchMuonOptimizer", "CoatStateMonarchMuon", "QuantizationConfig", "butterfly_blk",
           "butterfly_blk_op", "butterfly_blk_bwd_op", "patch_monarch_linear"]
