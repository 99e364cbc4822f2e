"""Synthetic workloads of the Monarch-Muon step (the benchmark configurations).

Parameter inventories follow the Monarch factor-shape rule
(``pretrain/src/models/monarch/monarch_linear.py:73-83``) over a LLaMA's
parameter order (``pretrain/src/models/llama.py:69-84,96-100,196-205``) and the
Muon/AdamW split of ``pretrain/src/main.py:156-165``.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, replace

import torch

VOCAB = 50304


@dataclass(frozen=True)
class Workload:
    name: str
    n_layer: int
    n_embd: int
    n_head: int
    intermediate: int
    nblocks: int
    param_dtype: torch.dtype
    momentum_dtype: torch.dtype | str     # torch dtype, or "fp8" for e4m3 states
    ns_dtype: torch.dtype | None          # None: Newton-Schulz in the momentum dtype
    prefill_momentum: bool                # momentum N(0, 1e-3) before step 1 (else zeros)
    shards: int = 1                       # > 1: one rank's share of a block-ownership sharded step


WORKLOADS = {
    # fp32 toy, momentum zero, pretrain semantics
    "toy": Workload("toy", 2, 512, 8, 1376, 2, torch.float32, torch.float32, None, False),
    # configs[1..3]: bf16 params/grads, fp32 momentum, bf16 Newton-Schulz
    "257m-nb2": Workload("257m-nb2", 24, 1024, 16, 2736, 2, torch.bfloat16, torch.float32, torch.bfloat16, True),
    "1.3b-nb4": Workload("1.3b-nb4", 24, 2048, 16, 5504, 4, torch.bfloat16, torch.float32, torch.bfloat16, True),
    "6.89b-nb4": Workload("6.89b-nb4", 32, 4096, 32, 11008, 4, torch.bfloat16, torch.float32, torch.bfloat16, True),
    # FP8 e4m3 momentum (group 128), bf16 Newton-Schulz
    "6.89b-nb4-fp8": Workload("6.89b-nb4-fp8", 32, 4096, 32, 11008, 4, torch.bfloat16, "fp8", torch.bfloat16, True),
    # the optimizer states the reference's published step time was measured with: bf16 params, grads and
    # momentum (membench/scripts/monarch_benchmark/benchmark_train_step.py:428-436 asserts bf16 states)
    "6.89b-nb4-bf16mom": Workload("6.89b-nb4-bf16mom", 32, 4096, 32, 11008, 4, torch.bfloat16, torch.bfloat16,
                                  torch.bfloat16, True),
    # the pretrain copy at 1.3B shapes: fp32 params, grads and momentum, Newton-Schulz in the momentum dtype
    # (pretrain/src/models/monarch/monarch_muon.py:133-165; the reference allows TF32 for these products,
    # pretrain/src/main.py:51)
    "1.3b-nb4-f32": Workload("1.3b-nb4-f32", 24, 2048, 16, 5504, 4, torch.float32, torch.float32, None, True),
    # one rank's share of the headline step sharded over 8 GPUs by block ownership: the Muon blocks of 4 of the
    # 32 layers (every layer has the same blocks, so whole layers balance the Newton-Schulz work) and 1/8 of the
    # AdamW group's elements (AdamW is elementwise; a rank owns a contiguous range of the flattened group)
    "6.89b-nb4-shard8": Workload("6.89b-nb4-shard8", 32, 4096, 32, 11008, 4, torch.bfloat16, torch.float32,
                                 torch.bfloat16, True, shards=8),
}


def mlp_hidden(n_embd: int, intermediate: int = 0, multiple_of: int = 256) -> int:
    if intermediate:
        return int(intermediate)
    h = int(2 * (n_embd * 4) / 3)
    return multiple_of * ((h + multiple_of - 1) // multiple_of)


def factor_shapes(d_in: int, d_out: int, nb: int):
    """(blkdiag1, blkdiag2) shapes of one Monarch linear."""
    ib, ob = math.ceil(d_in / nb), math.ceil(d_out / nb)
    if ib * nb < ob * nb:
        return (nb, ib, ib), (nb, ob, ib)
    return (nb, ob, ib), (nb, ob, ob)


def local_layers(w: Workload) -> int:
    """Transformer layers whose Muon blocks the workload holds (a rank's share when sharded)."""
    if w.n_layer % w.shards:
        raise ValueError(f"{w.name}: {w.n_layer} layers do not split over {w.shards} ranks")
    return w.n_layer // w.shards


def parameter_inventory(w: Workload):
    """Ordered ``[(name, shape, is_muon)]`` of the Monarch LLaMA's parameters.

    A sharded workload (``shards`` > 1) is rank 0's share: the Muon blocks of
    layers ``[0, n_layer / shards)`` and one flat tensor holding its
    ``ceil(1 / shards)`` range of the AdamW group's elements."""
    if w.shards > 1:
        full = replace(w, shards=1)
        share = -(-adamw_elements(full) // w.shards)
        muon = [(n, s, m) for n, s, m in parameter_inventory(full)
                if m and int(n.split(".")[2]) < local_layers(w)]
        return muon + [("adamw_group.elements_of_rank_0", (share,), False)]
    h, hid, nb = w.n_embd, mlp_hidden(w.n_embd, w.intermediate), w.nblocks
    out = [("transformer.wte.weight", (VOCAB, h))]
    for li in range(w.n_layer):
        pre = f"transformer.h.{li}"
        out.append((f"{pre}.ln_1.weight", (h,)))
        for nm in ("q_proj", "k_proj", "v_proj", "o_proj"):
            b1, b2 = factor_shapes(h, h, nb)
            out += [(f"{pre}.attn.{nm}.blkdiag1", b1), (f"{pre}.attn.{nm}.blkdiag2", b2)]
        out.append((f"{pre}.ln_2.weight", (h,)))
        for nm, (din, dout) in (("gate_proj", (h, hid)), ("up_proj", (h, hid)), ("down_proj", (hid, h))):
            b1, b2 = factor_shapes(din, dout, nb)
            out += [(f"{pre}.mlp.{nm}.blkdiag1", b1), (f"{pre}.mlp.{nm}.blkdiag2", b2)]
    out.append(("transformer.ln_f.weight", (h,)))
    out.append(("lm_head.weight", (VOCAB, h)))
    return [(n, s, len(s) >= 2 and not any(x in n for x in ("wte", "wpe", "lm_head", "embed")))
            for n, s in out]


def ns_flops(w: Workload, steps: int = 5) -> float:
    """Algorithmic Newton-Schulz FLOPs of one step: 2 m^2 (2n + m) per block and
    iteration (m = min(r, c), n = max(r, c))."""
    tot = 0.0
    for _, s, muon in parameter_inventory(w):
        if muon:
            m, n = min(s[1], s[2]), max(s[1], s[2])
            tot += s[0] * 2.0 * m * m * (2 * n + m) * steps
    return tot


def muon_elements(w: Workload) -> int:
    return sum(math.prod(s) for _, s, muon in parameter_inventory(w) if muon)


def adamw_elements(w: Workload) -> int:
    return sum(math.prod(s) for _, s, muon in parameter_inventory(w) if not muon)
