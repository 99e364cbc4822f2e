"""Monarch block shapes and parameter order, restated -- test infrastructure.

Restates:
* the factor-shape rule of ``MonarchLinear.__init__``
  (``pretrain/src/models/monarch/monarch_linear.py:73-83``);
* the LLaMA module order (``pretrain/src/models/llama.py:69-84,96-100,196-205``):
  ``wte``, then per layer ``ln_1, q, k, v, o, ln_2, gate, up, down``, then
  ``ln_f`` and ``lm_head``;
* the MLP width (``membench/src/models/llama.py:60-68``);
* the Muon/AdamW split of ``pretrain/src/main.py:156-165``.

Pinned by the exact parameter counts the reference's own test asserts
(``membench/tests/test_monarch_large_benchmark.py:95-112`` with
``membench/scripts/monarch_benchmark/common.py:13-64``).
"""
from __future__ import annotations

import math

VOCAB = 50304


def mlp_hidden(n_embd: int, intermediate: int = 0, multiple_of: int = 256) -> int:
    if intermediate:
        return int(intermediate)
    h = int(2 * (n_embd * 4) / 3)
    return multiple_of * ((h + multiple_of - 1) // multiple_of)


def monarch_factors(d_in: int, d_out: int, nb: int):
    ib = int(math.ceil(d_in / nb))
    ob = int(math.ceil(d_out / nb))
    if ib * nb < ob * nb:
        return (nb, ib, ib), (nb, ob, ib)
    return (nb, ob, ib), (nb, ob, ob)


def llama_monarch_params(n_layer, n_embd, intermediate, nb, vocab=VOCAB):
    """Ordered ``[(name, shape)]`` of a Monarch LLaMA's parameters."""
    hid = mlp_hidden(n_embd, intermediate)
    out = [("transformer.wte.weight", (vocab, n_embd))]
    for li in range(n_layer):
        pre = f"transformer.h.{li}"
        out.append((f"{pre}.ln_1.weight", (n_embd,)))
        for nm in ("q_proj", "k_proj", "v_proj", "o_proj"):
            b1, b2 = monarch_factors(n_embd, n_embd, nb)
            out += [(f"{pre}.attn.{nm}.blkdiag1", b1), (f"{pre}.attn.{nm}.blkdiag2", b2)]
        out.append((f"{pre}.ln_2.weight", (n_embd,)))
        for nm, (din, dout) in (("gate_proj", (n_embd, hid)), ("up_proj", (n_embd, hid)),
                                ("down_proj", (hid, n_embd))):
            b1, b2 = monarch_factors(din, dout, nb)
            out += [(f"{pre}.mlp.{nm}.blkdiag1", b1), (f"{pre}.mlp.{nm}.blkdiag2", b2)]
    out.append(("transformer.ln_f.weight", (n_embd,)))
    out.append(("lm_head.weight", (vocab, n_embd)))
    return out


def split_muon_adamw(named):
    """``main.py:156-165``: Muon = ndim>=2 and not an embedding/head."""
    muon, adamw = [], []
    for name, shape in named:
        if len(shape) >= 2 and not any(x in name for x in ("wte", "wpe", "lm_head", "embed")):
            muon.append((name, shape))
        else:
            adamw.append((name, shape))
    return muon, adamw
