"""Write golden vectors of the reference Monarch-Muon step (run in the build
container, where the reference checkout exists).

The reference module files import only ``math``, ``collections`` and ``torch``;
they are loaded by path (not through their package, whose ``__init__`` pulls
in Triton).  Inputs are regenerated from the seed by ``tests/golden_inputs.py``
(the same generator the tests use), so the fixture holds the outputs plus a
checksum of the inputs.

    python tests/golden/make_golden.py /root/reference
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
from golden_inputs import CASES, make_case, input_checksum  # noqa: E402


def load(path: Path, name: str):
    spec = importlib.util.spec_from_file_location(name, path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def main(ref_root: str) -> None:
    root = Path(ref_root)
    mods = {
        "membench": load(root / "membench/src/models/monarch/monarch_muon.py", "ref_membench_monarch_muon"),
        "pretrain": load(root / "pretrain/src/models/monarch/monarch_muon.py", "ref_pretrain_monarch_muon"),
    }
    torch.set_num_threads(1)
    for case in CASES:
        mod = mods[case["variant"]]
        muon, adamw, bufs = make_case(case)
        opt = mod.MonarchMuonOptimizer(muon, adamw, lr=case["lr"], momentum=0.95,
                                       adamw_betas=(0.9, 0.95), adamw_weight_decay=0.1, adamw_eps=1e-8)
        if bufs is not None:
            for p, b in zip(muon, bufs):
                opt.state[p]["momentum_buffer"] = b
        out = {"inputs_sha": input_checksum(case)}
        for step in range(case["steps"]):
            opt.step()
        out["muon_params"] = [p.detach().clone() for p in muon]
        out["momentum"] = [opt.state[p]["momentum_buffer"].clone() for p in muon]
        out["adamw_params"] = [p.detach().clone() for p in adamw]
        out["exp_avg"] = [opt.state[p]["exp_avg"].clone() for p in adamw]
        out["exp_avg_sq"] = [opt.state[p]["exp_avg_sq"].clone() for p in adamw]
        # Newton-Schulz output of the case's first stack, as the reference computes it
        stack = torch.cat([b.clone() for b in (bufs or [torch.zeros_like(muon[0])])[:1]], 0)
        if case["variant"] == "membench":
            stack = stack.to(torch.bfloat16)
        out["ns_input"] = stack
        out["ns_output"] = mod._newton_schulz_batched(stack)
        torch.save(out, HERE / f"{case['name']}.pt")
        print("wrote", case["name"])


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
