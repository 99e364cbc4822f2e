"""The optimizer API the reference's callers use, on the GPU.

- ``step(closure)`` evaluates the closure with gradients enabled and returns
  its loss (membench ``monarch_muon.py:114-128``);
- under ``LambdaLR`` (``pretrain/src/optim/utils.py:63-72``) every group gains
  ``initial_lr`` and an lr changed between steps reaches the kernels;
- resume (``pretrain/src/optim/utils.py:103-132``; FP8 states:
  ``pretrain/tests/test_coat_state_muon.py:80-97``): a state_dict saved after
  step 2 and loaded into a fresh optimizer gives a step 3 bit-identical to the
  uninterrupted run's.
"""
import io

import pytest
import torch

from golden_inputs import CASES, make_case
from monarch_muon_amd import CoatStateMonarchMuon, MonarchMuonOptimizer, QuantizationConfig

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _opt(case, muon, adamw, fp8, lr=0.02):
    ns = torch.bfloat16 if case["variant"] == "membench" else None
    if fp8:
        return CoatStateMonarchMuon(muon, adamw, lr=lr, momentum=0.95, qargs=QuantizationConfig(), ns_dtype=ns)
    return MonarchMuonOptimizer(muon, adamw, lr=lr, momentum=0.95, ns_dtype=ns)


def _bits(t):
    return t.view(torch.uint8) if t.dtype == torch.float8_e4m3fn else t


def test_step_closure_returns_loss_and_uses_its_gradients():
    case = CASES[1]
    muon, adamw, _ = make_case(case, device=DEV)
    m2, a2, _ = make_case(case, device=DEV)
    for p in muon + adamw:
        p.grad = None
    calls = []

    def closure():
        assert torch.is_grad_enabled()
        loss = sum((p.float() ** 2).sum() for p in muon + adamw)
        loss.backward()
        calls.append(1)
        return loss

    opt = MonarchMuonOptimizer(muon, adamw, lr=0.02)
    loss = opt.step(closure)
    assert calls == [1] and torch.is_tensor(loss) and loss.requires_grad
    # the same step with the closure's gradients computed beforehand
    for p in m2 + a2:
        p.grad = None
    with torch.enable_grad():
        ref_loss = sum((p.float() ** 2).sum() for p in m2 + a2)
        ref_loss.backward()
    ref = MonarchMuonOptimizer(m2, a2, lr=0.02)
    assert ref.step() is None
    torch.cuda.synchronize()
    assert torch.equal(loss.detach(), ref_loss.detach())
    for p, q in zip(muon + adamw, m2 + a2):
        assert torch.equal(p, q)


@pytest.mark.parametrize("fp8", [False, True], ids=["plain", "fp8"])
def test_lambda_lr_schedule_reaches_the_kernels(fp8):
    case = CASES[1]
    factors = [1.0, 0.5, 0.25]
    muon, adamw, _ = make_case(case, device=DEV)
    opt = _opt(case, muon, adamw, fp8)
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: factors[min(s, len(factors) - 1)])
    assert all(g["initial_lr"] == 0.02 for g in opt.param_groups)
    sd = opt.state_dict()
    assert all(g["initial_lr"] == 0.02 for g in sd["param_groups"])
    m2, a2, _ = make_case(case, device=DEV)
    ref = _opt(case, m2, a2, fp8)
    for f in factors:
        assert all(g["lr"] == pytest.approx(0.02 * f) for g in opt.param_groups)
        opt.step()
        sched.step()
        for g in ref.param_groups:
            g["lr"] = 0.02 * f
        ref.step()
    torch.cuda.synchronize()
    for p, q in zip(muon + adamw, m2 + a2):
        assert torch.equal(p, q)
    # a different lr gives different weights: the value is not ignored
    m3, a3, _ = make_case(case, device=DEV)
    other = _opt(case, m3, a3, fp8)
    for _ in factors:
        other.step()
    torch.cuda.synchronize()
    assert not torch.equal(muon[0], m3[0])


@pytest.mark.parametrize("case_idx,fp8", [(1, False), (2, False), (1, True), (2, True)],
                         ids=["membench-bf16", "pretrain-fp32", "membench-bf16-fp8", "pretrain-fp32-fp8"])
def test_resume_after_step_two_equals_uninterrupted(case_idx, fp8):
    case = CASES[case_idx]
    muon, adamw, _ = make_case(case, device=DEV)
    opt = _opt(case, muon, adamw, fp8)
    sched = torch.optim.lr_scheduler.LambdaLR(opt, lambda s: 1.0 / (1 + s))
    for _ in range(2):
        opt.step()
        sched.step()
    torch.cuda.synchronize()
    snapshot = [p.detach().clone() for p in muon + adamw]
    buf = io.BytesIO()
    torch.save({"optimizer": opt.state_dict(), "scheduler": sched.state_dict()}, buf)
    opt.step()                                              # uninterrupted step 3
    torch.cuda.synchronize()

    buf.seek(0)
    ckpt = torch.load(buf, weights_only=True)
    m2, a2, _ = make_case(case, device=DEV)
    with torch.no_grad():
        for p, s in zip(m2 + a2, snapshot):
            p.copy_(s)
    opt2 = _opt(case, m2, a2, fp8)
    sched2 = torch.optim.lr_scheduler.LambdaLR(opt2, lambda s: 1.0 / (1 + s))
    opt2.load_state_dict(ckpt["optimizer"])
    sched2.load_state_dict(ckpt["scheduler"])
    assert [g["lr"] for g in opt2.param_groups] == [g["lr"] for g in opt.param_groups]
    opt2.step()                                             # resumed step 3
    torch.cuda.synchronize()
    for p, q in zip(muon + adamw, m2 + a2):
        assert torch.equal(p, q)
    for p, q in zip(muon + adamw, m2 + a2):
        s1, s2 = opt.state[p], opt2.state[q]
        assert set(s1) == set(s2)
        for k in s1:
            if torch.is_tensor(s1[k]):
                assert s1[k].dtype == s2[k].dtype, k
                assert torch.equal(_bits(s1[k]), _bits(s2[k])), k
            else:
                assert s1[k] == s2[k], k


@pytest.mark.parametrize("case_idx,fp8", [(0, False), (1, True)], ids=["bf16-fp32mom", "bf16-fp8"])
def test_fresh_gradient_tensors_each_step_equal_fixed_ones(case_idx, fp8):
    """A training loop drops its gradients after every step
    (``zero_grad(set_to_none=True)``, ``pretrain/src/optim/base.py:125``) and
    the next backward allocates new ones: the planners then rewrite only the
    gradient column of their tables.  Three steps with new gradient tensors at
    new addresses (the old ones still alive, so no address is reused) must give
    the bits of three steps with one fixed set of gradient tensors."""
    case = CASES[case_idx]
    m1, a1, b1 = make_case(case, device=DEV)
    m2, a2, b2 = make_case(case, device=DEV)
    o1, o2 = _opt(case, m1, a1, fp8), _opt(case, m2, a2, fp8)
    if b1 is not None and not fp8:
        for p, q, x, y in zip(m1, m2, b1, b2):
            o1.state[p]["momentum_buffer"], o2.state[q]["momentum_buffer"] = x, y
    held = []
    for step in range(3):
        old = [p.grad for p in m1 + a1]
        held.append(old)
        for p, g in zip(m1 + a1, old):
            p.grad = g * (1.0 + 0.25 * step)        # a new tensor at a new address
        for p, q in zip(m1 + a1, m2 + a2):
            q.grad.copy_(p.grad)                    # the same values in the fixed tensors
        o1.step()
        o2.step()
    torch.cuda.synchronize()
    for p, q in zip(m1 + a1, m2 + a2):
        assert torch.equal(p, q)
        s1, s2 = o1.state[p], o2.state[q]
        for k in s1:
            if torch.is_tensor(s1[k]):
                assert torch.equal(_bits(s1[k]), _bits(s2[k])), k
    # a fourth step with a non-contiguous gradient (same values): it is read
    # through a contiguous copy, on the gradient-only path as well
    g = m1[0].grad
    nc = torch.empty(g.shape[0], g.shape[2], g.shape[1], dtype=g.dtype, device=DEV).transpose(1, 2)
    nc.copy_(g)
    assert not nc.is_contiguous()
    m1[0].grad = nc
    o1.step()
    o2.step()
    torch.cuda.synchronize()
    for p, q in zip(m1 + a1, m2 + a2):
        assert torch.equal(p, q)


def _layer(name, seed=3):
    """One layer's Monarch factors of a workload (bf16 params and grads) and a
    short AdamW tensor, drawn on the GPU."""
    from monarch_muon_amd.workloads import WORKLOADS, parameter_inventory
    w = WORKLOADS[name]
    gen = torch.Generator(device=DEV).manual_seed(seed)
    muon, adamw = [], []
    for n, s, is_muon in parameter_inventory(w):
        if is_muon and (".h." not in n or int(n.split(".")[2]) > 0):
            continue
        if not is_muon:
            s = (64,) + tuple(s[1:]) if len(s) == 2 else s
        p = (torch.randn(s, generator=gen, device=DEV) * 0.02).bfloat16()
        p.grad = (torch.randn(s, generator=gen, device=DEV) * 1e-3).bfloat16()
        (muon if is_muon else adamw).append(p)
    return muon, adamw[:2]


@pytest.mark.parametrize("fp8", [False, True], ids=["fp32mom", "fp8"])
@pytest.mark.parametrize("name", ["1.3b-nb4", "6.89b-nb4"])
def test_shared_newton_schulz_launches_equal_per_group_launches(name, fp8):
    """Groups of one Newton-Schulz geometry (a tall group and its wide
    counterpart, e.g. 2752 x 1024 and 1024 x 2752) share every launch but the
    apply; two steps that way give the bits of two steps with each group
    launched on its own (the reference's one batch per shape)."""
    from monarch_muon_amd.plan import BatchLaunch
    m1, a1 = _layer(name)
    m2, a2 = _layer(name)
    mk = (lambda m, a: CoatStateMonarchMuon(m, a, lr=0.02, momentum=0.95, qargs=QuantizationConfig())) if fp8 \
        else (lambda m, a: MonarchMuonOptimizer(m, a, lr=0.02, momentum=0.95))
    o1, o2 = mk(m1, a1), mk(m2, a2)
    o2._muon_planner.merge = False
    if not fp8:
        gen = torch.Generator(device=DEV).manual_seed(9)
        for p, q in zip(m1, m2):
            b = torch.randn(p.shape, generator=gen, device=DEV) * 1e-3
            o1.state[p]["momentum_buffer"], o2.state[q]["momentum_buffer"] = b, b.clone()
    for _ in range(2):
        o1.step()
        o2.step()
    torch.cuda.synchronize()
    batches = [u for u in o1._muon_planner.units if isinstance(u, BatchLaunch)]
    assert [[(g.rows, g.cols) for g in b.members] for b in batches] == \
        ([[(1376, 512), (512, 1376)]] if name == "1.3b-nb4" else [[(2752, 1024), (1024, 2752)]])
    assert not any(isinstance(u, BatchLaunch) for u in o2._muon_planner.units)
    for p, q in zip(m1 + a1, m2 + a2):
        assert torch.equal(p, q)
        s1, s2 = o1.state[p], o2.state[q]
        for k in s1:
            if torch.is_tensor(s1[k]):
                assert torch.equal(_bits(s1[k]), _bits(s2[k])), k


@pytest.mark.parametrize("fp8", [False, True], ids=["fp32mom", "fp8"])
def test_steps_on_side_streams_equal_default_stream(fp8):
    """The reference's benchmark harness builds its states and runs
    ``optimizer.step()`` inside ``with torch.cuda.stream(stream)`` on a stream of
    its own (``membench/scripts/monarch_benchmark/benchmark_train_step.py:285-299,
    382``).  Here the optimizer is built and stepped on one side stream, the
    next step runs on a second one and the third on the default stream (each
    stream waiting on the previous one, as any program that moves work
    between streams does); the planners' table uploads, workspaces and FP8
    metadata follow the current stream.  The bits equal three steps on the
    default stream."""
    def run(streams):
        muon, adamw = _layer("1.3b-nb4", seed=5)
        prev = torch.cuda.current_stream()
        opt = None
        for s in streams:
            s = s or torch.cuda.default_stream(DEV)
            s.wait_stream(prev)
            with torch.cuda.stream(s):
                if opt is None:
                    opt = (CoatStateMonarchMuon(muon, adamw, lr=0.02, momentum=0.95, qargs=QuantizationConfig())
                           if fp8 else MonarchMuonOptimizer(muon, adamw, lr=0.02, momentum=0.95))
                    if not fp8:
                        gen = torch.Generator(device=DEV).manual_seed(9)
                        for p in muon:
                            opt.state[p]["momentum_buffer"] = torch.randn(p.shape, generator=gen, device=DEV) * 1e-3
                for p in muon + adamw:   # the next step's gradients, written on this stream
                    p.grad.mul_(1.25)
                opt.step()
            prev = s
        torch.cuda.default_stream(DEV).wait_stream(prev)
        torch.cuda.synchronize()
        return muon + adamw, opt

    s1, s2 = torch.cuda.Stream(DEV), torch.cuda.Stream(DEV)   # default priority
    ref, ropt = run([None, None, None])
    got, gopt = run([s1, s2, None])
    for p, q in zip(ref, got):
        assert torch.equal(p, q)
        st1, st2 = ropt.state[p], gopt.state[q]
        assert set(st1) == set(st2)
        for k in st1:
            if torch.is_tensor(st1[k]):
                assert torch.equal(_bits(st1[k]), _bits(st2[k])), k


def test_group_with_mixed_parameter_dtypes_matches_oracle():
    """The reference keys its groups on the momentum buffer (device, dtype,
    rows, cols) and applies the update per parameter (membench
    ``monarch_muon.py:156,165-170``), so one group may hold bf16 and fp32
    parameters whose buffers are both fp32.  Such a group gets one launch
    group per (param, grad) dtype pair sharing its Newton-Schulz launches; the
    step matches the oracle (weights within the bf16 bar, momentum bit for
    bit)."""
    from monarch_muon_amd.plan import BatchLaunch
    from oracle.step import ReferenceMonarchMuon
    from test_gpu_parity import BF16_TOL, blocks_rel
    gen = torch.Generator().manual_seed(41)
    spec = [((2, 256, 256), torch.bfloat16), ((1, 256, 256), torch.float32), ((1, 256, 256), torch.bfloat16),
            ((2, 688, 256), torch.float32), ((1, 688, 256), torch.bfloat16)]
    draws = [(torch.randn(s, generator=gen) * 0.02, torch.randn(s, generator=gen) * 1e-3,
              torch.randn(s, generator=gen) * 1e-3, dt) for s, dt in spec]

    def build(device, cls, **kw):
        ps = []
        for w, g, _, dt in draws:
            p = w.to(dt).to(device).requires_grad_(True)
            p.grad = g.to(dt).to(device)
            ps.append(p)
        opt = cls(ps, [], lr=0.02, momentum=0.95, **kw)
        for p, (_, _, b, _) in zip(ps, draws):
            opt.state[p]["momentum_buffer"] = b.to(device)   # fp32 buffers for every parameter
        return ps, opt

    gp, gopt = build(DEV, MonarchMuonOptimizer)
    cp, copt = build("cpu", ReferenceMonarchMuon, variant="membench")
    for _ in range(2):
        gopt.step()
        copt.step()
    torch.cuda.synchronize()
    groups = gopt._muon_planner.groups
    assert [(g.rows, g.cols, g.nblocks, g.struct.param_dtype) for g in groups] == \
        [(256, 256, 3, 1), (256, 256, 1, 0), (688, 256, 2, 0), (688, 256, 1, 1)]
    batches = [u for u in gopt._muon_planner.units if isinstance(u, BatchLaunch)]
    assert [[(g.rows, g.nblocks) for g in b.members] for b in batches] == [[(256, 3), (256, 1)], [(688, 2), (688, 1)]]
    for p, q in zip(gp, cp):
        assert p.dtype == q.dtype
        assert blocks_rel(p, q).max() <= BF16_TOL
        assert torch.equal(gopt.state[p]["momentum_buffer"].cpu(), copt.state[q]["momentum_buffer"])
