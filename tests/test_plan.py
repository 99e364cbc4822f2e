"""Planner and workload inventories against the oracle's independent restatement
and the closed-form block counts (CPU)."""
import math
from collections import OrderedDict

import pytest
import torch

from monarch_muon_amd.plan import adamw_scalars, group_key, plan_groups
from monarch_muon_amd.workloads import WORKLOADS, adamw_elements, muon_elements, ns_flops, parameter_inventory
from oracle import shapes
from oracle.step import group_blocks

# (muon tensors, muon elements, [(rows, cols, blocks)], adamw elements, NS TFLOP 3-product form)
APPENDIX_B = {
    "toy": (28, 4_997_120, [(256, 256, 44), (688, 256, 8), (256, 688, 4)], 51_513_856, 0.035),
    "257m-nb2": (336, 239_271_936, [(512, 512, 528), (1368, 512, 96), (512, 1368, 48)], 103_072_768, 3.35),
    "1.3b-nb4": (336, 479_723_520, [(512, 512, 1056), (1376, 512, 192), (512, 1376, 96)], 206_145_536, 6.72),
    "6.89b-nb4": (448, 2_558_525_440, [(1024, 1024, 1408), (2752, 1024, 256), (1024, 2752, 128)],
                  412_356_608, 71.64),
}


@pytest.mark.parametrize("name", list(APPENDIX_B))
def test_inventory_matches_closed_form_and_oracle(name):
    w = WORKLOADS[name]
    inv = parameter_inventory(w)
    ours = [(n, s) for n, s, _ in inv]
    ref = shapes.llama_monarch_params(w.n_layer, w.n_embd, w.intermediate, w.nblocks)
    assert ours == ref
    mu_ref, ad_ref = shapes.split_muon_adamw(ref)
    assert [(n, s) for n, s, m in inv if m] == mu_ref
    n_t, n_el, groups, n_ad, tflop = APPENDIX_B[name]
    assert len(mu_ref) == n_t and muon_elements(w) == n_el and adamw_elements(w) == n_ad
    # planner grouping == reference grouping, in order
    bufs = [torch.empty(s, device="meta") for _, s in mu_ref]
    planned = [(k[2], k[3], sum(bufs[i].shape[0] for i in idx)) for k, idx in plan_groups(bufs).items()]
    assert planned == groups
    oracle_groups = [(k[2], k[3], sum(b.shape[0] for _, _, b in items))
                     for k, items in group_blocks(bufs, bufs).items()]
    assert planned == oracle_groups
    assert abs(ns_flops(w) / 1e12 - tflop) < 0.006


def test_plan_groups_preserves_member_order():
    bufs = [torch.empty(2, 8, 8), torch.empty(1, 16, 8), torch.empty(3, 8, 8), torch.empty(1, 8, 16),
            torch.empty(1, 16, 8, dtype=torch.bfloat16)]
    g = plan_groups(bufs)
    assert list(g.values()) == [[0, 2], [1], [3], [4]]
    assert list(g.keys())[0] == group_key(bufs[0])


def test_plan_groups_rejects_non_3d():
    with pytest.raises(ValueError):
        plan_groups([torch.empty(4, 4)])


def test_adamw_scalars_are_python_doubles():
    s = adamw_scalars(1e-3, 0.9, 0.95, 1e-8, 0.1, 3)
    assert s["neg_step_size"] == -1e-3 / (1 - 0.9 ** 3)
    assert s["sqrt_bc2"] == math.sqrt(1 - 0.95 ** 3)
    assert s["wd_factor"] == 1 - 1e-3 * 0.1 and s["apply_weight_decay"] == 1
    assert adamw_scalars(1e-3, 0.9, 0.95, 1e-8, 0.0, 1)["apply_weight_decay"] == 0


def test_shard_workload_is_one_eighth_of_the_headline_step():
    """Rank 0's share of an 8-way block-ownership step: the Muon blocks of 4 of
    the 32 layers (one eighth of every shape group, in the same order) and one
    eighth of the AdamW elements; one eighth of the Newton-Schulz work."""
    full, shard = WORKLOADS["6.89b-nb4"], WORKLOADS["6.89b-nb4-shard8"]
    inv = parameter_inventory(shard)
    mu = [s for _, s, m in inv if m]
    bufs = [torch.empty(s, device="meta") for s in mu]
    planned = [(k[2], k[3], sum(bufs[i].shape[0] for i in idx)) for k, idx in plan_groups(bufs).items()]
    assert planned == [(r, c, n // 8) for r, c, n in APPENDIX_B["6.89b-nb4"][2]]
    assert [n for n, _, m in inv if m] == [n for n, _, m in parameter_inventory(full) if m][: len(mu)]
    assert muon_elements(shard) * 8 == muon_elements(full)
    assert adamw_elements(shard) == -(-adamw_elements(full) // 8)
    assert abs(ns_flops(shard) * 8 - ns_flops(full)) < 1e3
