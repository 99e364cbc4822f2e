"""Gradient-norm clipping folded into the step (``clip_grad_norm_`` on the
optimizer) against what the reference runs: ``torch.nn.utils.clip_grad_norm_``
over the model's parameters, then ``opt.step()`` (pretrain/src/optim/base.py:121-122).

torch rescales ``p.grad`` in place by ``min(max_norm / (total + 1e-6), 1)`` in the
gradients' dtype; the fused path leaves the gradients alone and the step reads
``dtype(g * coef)``.  With the same coefficient the two steps are bit-identical.
The total norm is an fp32 reduction in both, in different orders, rounded to the
gradients' dtype, so it can differ only where the fp32 sums straddle a rounding
boundary of that dtype (never for the bf16 cases here; fp32 gets a tolerance).
"""
import pytest
import torch

from golden_inputs import CASES, make_case
from monarch_muon_amd import CoatStateMonarchMuon, MonarchMuonOptimizer, QuantizationConfig
from oracle.step import ReferenceMonarchMuon
from oracle.truth import rel_fro

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
BF16_TOL, F32_TOL = 1e-2, 1e-5


def blocks_rel(a, b):
    a, b = a.detach().cpu().double(), b.detach().cpu().double()
    if a.dim() < 3:
        a, b = a.reshape(1, 1, -1), b.reshape(1, 1, -1)
    return rel_fro(a, b)


def _opt(case, device, cls=MonarchMuonOptimizer, **kw):
    muon, adamw, bufs = make_case(case, device=device)
    if cls is ReferenceMonarchMuon:
        opt = cls(muon, adamw, lr=case["lr"], momentum=0.95, variant=case["variant"])
    else:
        kw.setdefault("ns_dtype", torch.bfloat16 if case["variant"] == "membench" else None)
        opt = cls(muon, adamw, lr=case["lr"], momentum=0.95, **kw)
    if bufs is not None and cls is not CoatStateMonarchMuon:
        for p, b in zip(muon, bufs):
            opt.state[p]["momentum_buffer"] = b
    return muon, adamw, opt


def _total_norm(case):
    muon, adamw, _ = make_case(case, device=DEV)
    return float(torch.nn.utils.clip_grad_norm_(muon + adamw, 1e30))


@pytest.mark.parametrize("clip", ["clips", "no-op"])
@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_fused_clip_equals_torch_clip_then_step(case, clip):
    max_norm = 0.25 * _total_norm(case) if clip == "clips" else 10.0 * _total_norm(case)
    ma, aa, oa = _opt(case, DEV)
    ta = torch.nn.utils.clip_grad_norm_(ma + aa, max_norm)
    oa.step()
    mb, ab, ob = _opt(case, DEV)
    before = [p.grad.clone() for p in mb + ab]
    tb = ob.clip_grad_norm_(max_norm)
    ob.step()
    torch.cuda.synchronize()
    assert tb.dtype == ta.dtype and tb.dim() == 0
    for g0, p in zip(before, mb + ab):
        assert torch.equal(g0, p.grad), "the fused path must not rewrite the gradients"
    assert ob._clip is None, "a clipping coefficient applies to one step only"
    same = torch.equal(tb.cpu(), ta.cpu())
    if case["dtype"] == torch.bfloat16:
        assert same, (tb.item(), ta.item())
    else:
        assert abs(tb.item() - ta.item()) <= 2e-7 * abs(ta.item())
    tol = BF16_TOL if case["variant"] == "membench" else F32_TOL
    for p, q in zip(ma + aa, mb + ab):
        if same:
            assert torch.equal(p, q)
        else:
            assert blocks_rel(p, q).max() <= tol
    for p, q in zip(ma, mb):
        if same:
            assert torch.equal(oa.state[p]["momentum_buffer"], ob.state[q]["momentum_buffer"])


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_fused_clip_step_matches_oracle(case):
    max_norm = 0.25 * _total_norm(case)
    gm, ga, gopt = _opt(case, DEV)
    gopt.clip_grad_norm_(max_norm)
    gopt.step()
    cm, ca, copt = _opt(case, "cpu", ReferenceMonarchMuon)
    torch.nn.utils.clip_grad_norm_(cm + ca, max_norm)
    copt.step()
    torch.cuda.synchronize()
    tol = BF16_TOL if case["variant"] == "membench" else F32_TOL
    for p, q in zip(gm + ga, cm + ca):
        assert blocks_rel(p, q).max() <= tol


def test_fused_clip_fp8_states():
    case = CASES[0]
    max_norm = 0.25 * _total_norm(case)
    ma, aa, oa = _opt(case, DEV, CoatStateMonarchMuon, qargs=QuantizationConfig())
    torch.nn.utils.clip_grad_norm_(ma + aa, max_norm)
    oa.step()
    mb, ab, ob = _opt(case, DEV, CoatStateMonarchMuon, qargs=QuantizationConfig())
    ob.clip_grad_norm_(max_norm)
    ob.step()
    torch.cuda.synchronize()
    for p, q in zip(ma + aa, mb + ab):
        assert torch.equal(p, q)
    for p, q in zip(ma, mb):
        assert torch.equal(oa.state[p]["momentum_buffer"].view(torch.uint8),
                           ob.state[q]["momentum_buffer"].view(torch.uint8))


def test_fused_clip_cleared_by_zero_grad_and_repeatable():
    case = CASES[0]
    mb, ab, ob = _opt(case, DEV)
    t1 = ob.clip_grad_norm_(1e-3)
    t2 = ob.clip_grad_norm_(1e-3)
    assert torch.equal(t1, t2)
    ob.zero_grad()
    assert ob._clip is None
    with pytest.raises(NotImplementedError):
        ob.clip_grad_norm_(1.0, norm_type=1.0)
