"""CPU oracle for the Monarch-Muon optimizer step -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference implementation of the one hot
path this repository accelerates (``MonarchMuonOptimizer.step()`` of
brain-lab-research/monarch-muon).  It exists to CHECK the HIP implementation in
``monarch_muon_amd``; nothing in the product path may import it.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker / the timed CPU baseline.

Modules
-------
step    torch-CPU restatement of the optimizer step (both reference copies:
        the bf16-Newton-Schulz ``membench`` copy and the buffer-dtype
        ``pretrain`` copy), the block grouping, and the embedded AdamW.
codec   numpy restatement of the FP8 (e4m3, group-128, dynamic range
        expansion) state codec of ``coat_state_muon.py``.
shapes  the Monarch block-shape rule and LLaMA parameter order, restated.
truth   fp64 closed forms used to pin the restatement (scalar quintic, SVD
        known-answer, invariants).

Pinning status (what each function is checked against) is stated in each
module header; every function is pinned by at least one check in
``tests/test_oracle.py`` that a dropped term, a wrong sign or a transposed
operand would fail.
"""
