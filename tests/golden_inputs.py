"""Seeded inputs of the golden-vector cases (shared by the fixture writer and the tests).

Draw order: for each Muon parameter W ~ N(0, 0.02), g ~ N(0, 1e-3), then (if
prefilled) buf ~ N(0, 1e-3); then for each AdamW parameter W ~ N(0, 0.02),
g ~ N(0, 1e-3).  Everything is drawn in fp32 on the CPU from one
``torch.Generator`` and then cast, so every consumer sees identical bits.
"""
from __future__ import annotations

import hashlib

import torch

# square, tall, wide, square again (first-appearance grouping), tall again
MUON_SHAPES = [(2, 64, 64), (1, 128, 64), (1, 64, 128), (1, 64, 64), (1, 128, 64), (1, 96, 136), (1, 136, 96)]
ADAMW_SHAPES = [(100, 64), (64,), (37,)]

CASES = [
    dict(name="membench_bf16_fp32mom", variant="membench", dtype=torch.bfloat16, mom=torch.float32,
         prefill=True, lr=0.02, steps=2, seed=0),
    dict(name="membench_bf16_bf16mom", variant="membench", dtype=torch.bfloat16, mom=None,
         prefill=False, lr=0.02, steps=2, seed=1),
    dict(name="pretrain_fp32", variant="pretrain", dtype=torch.float32, mom=None,
         prefill=False, lr=0.02, steps=2, seed=2),
]


def _draws(case):
    g = torch.Generator().manual_seed(case["seed"])
    out = []
    for s in MUON_SHAPES:
        out.append(torch.randn(s, generator=g) * 0.02)
        out.append(torch.randn(s, generator=g) * 1e-3)
        if case["prefill"]:
            out.append(torch.randn(s, generator=g) * 1e-3)
    for s in ADAMW_SHAPES:
        out.append(torch.randn(s, generator=g) * 0.02)
        out.append(torch.randn(s, generator=g) * 1e-3)
    return out


def input_checksum(case) -> str:
    h = hashlib.sha256()
    for t in _draws(case):
        h.update(t.numpy().tobytes())
    return h.hexdigest()


def make_case(case, device="cpu"):
    """``(muon_params, adamw_params, momentum_buffers or None)`` with grads set."""
    d = iter(_draws(case))
    dt = case["dtype"]
    muon, adamw, bufs = [], [], []
    for _ in MUON_SHAPES:
        w = next(d).to(dt).to(device).requires_grad_(True)
        w.grad = next(d).to(dt).to(device)
        muon.append(w)
        if case["prefill"]:
            bufs.append(next(d).to(case["mom"]).to(device))
    for _ in ADAMW_SHAPES:
        w = next(d).to(dt).to(device).requires_grad_(True)
        w.grad = next(d).to(dt).to(device)
        adamw.append(w)
    return muon, adamw, (bufs if case["prefill"] else None)
