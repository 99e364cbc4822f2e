"""The Newton-Schulz launch plans of libmmuon (``mmuon_ns_plan``, host-only)
executed on the CPU (no GPU calls).

Each plan op is carried out with torch matrix products over a model of the
workspace memory: writing a buffer destroys every buffer that shares its
storage (an X stack and its two m x m sub-stacks), and reading a destroyed
buffer fails the test.  Pins:

- in fp64 every plan equals the fp64 Newton-Schulz iteration (the reference's
  quintic, ``oracle.truth.ns_fp64``) to rounding: a wrong product order, a
  missing or doubled normalisation, an operand of the wrong iteration or a
  buffer overwritten while still needed fails by orders of magnitude;
- with every op's output rounded to bf16 (fp64 accumulation), as the bf16
  kernels round, the Gram form stays within the GPU tests' bar (1.5x the
  reference's own bf16 error against fp64, +2e-3) on blocks whose singular
  values span decades -- the case that rules out the Gram recursion without its
  rebuild of X;
- eligibility: the Gram form only for bf16 groups whose padded long side is at
  least twice the short one, five iterations, and not under MMUON_NS_STANDARD.
"""
import pytest
import torch

from monarch_muon_amd import _abi
from oracle.step import NS_COEFFS, NS_EPS, newton_schulz_batched
from oracle.truth import ns_fp64, rel_fro

A_C, B_C, C_C = NS_COEFFS
HOME = {_abi.NSB_X0_S0: _abi.NSB_X0, _abi.NSB_X0_S1: _abi.NSB_X0,
        _abi.NSB_X1_S0: _abi.NSB_X1, _abi.NSB_X1_S1: _abi.NSB_X1}


def _sharing(b):
    """Buffers whose storage overlaps b's (b excluded): an X stack and its two
    sub-stacks overlap; the two sub-stacks of one X stack do not."""
    if b in HOME:
        return {HOME[b]}
    return {k for k, h in HOME.items() if h == b}


def run_plan(ops, x0, rnd=lambda t: t):
    """Execute a plan on a (m x n) block x0 (the packed X, unnormalised; rows m
    <= n).  ``rnd`` rounds every op output (bf16 emulation).  Returns the final
    X (NO_APPLY plans) or the update U the apply adds (apply plans)."""
    m = x0.shape[0]
    s = 1.0 / (float(torch.linalg.matrix_norm(x0)) + NS_EPS)
    mem = {_abi.NSB_X0: x0}
    eye = torch.eye(m, dtype=x0.dtype)

    def get(b):
        assert b in mem, f"op reads buffer {b}, which a later write destroyed or nothing wrote"
        return mem[b]

    def put(b, v):
        for k in _sharing(b):
            mem.pop(k, None)
        mem[b] = rnd(v)

    for op in ops:
        f = s if op.scaled else 1.0
        if op.kind == _abi.NSOP_SYRK:
            x = get(op.in0)
            put(op.out, (f * f) * (x @ x.T))
        elif op.kind == _abi.NSOP_POLY:
            a = get(op.in0)
            put(op.out, A_C * eye + B_C * a + C_C * (a @ a))
        elif op.kind == _abi.NSOP_SYMM:
            put(op.out, get(op.in0) @ get(op.in1))
        elif op.kind == _abi.NSOP_PX:
            put(op.out, f * (get(op.in0) @ get(op.in1)))
        elif op.kind == _abi.NSOP_PX_APPLY:
            assert op is ops[-1] and op.out == _abi.NSB_PARAM
            return rnd(f * (get(op.in0) @ get(op.in1)))
        else:
            raise AssertionError(f"unknown op kind {op.kind}")
    return mem[ops[-1].out]


def bf16(t):
    return t.to(torch.bfloat16).to(t.dtype)


def kinds(ops):
    return [op.kind for op in ops]


GRAM_SHAPES = [(1024, 2752), (2752, 1024), (512, 1376), (1376, 512), (512, 1368), (256, 688)]
STANDARD_SHAPES = [(1024, 1024), (512, 512), (96, 136), (136, 96), (256, 256)]


@pytest.mark.parametrize("rows,cols", GRAM_SHAPES + STANDARD_SHAPES)
def test_plan_form_and_eligibility(rows, cols):
    lay = _abi.ns_layout(rows, cols, _abi.BF16, 1)
    gram = lay.np_ >= 2 * lay.mp
    assert gram == ((rows, cols) in GRAM_SHAPES)
    ops = _abi.ns_plan(rows, cols, _abi.BF16, 5)
    std = _abi.ns_plan(rows, cols, _abi.BF16, 5, _abi.NS_STANDARD)
    chain = [_abi.NSOP_SYRK, _abi.NSOP_POLY, _abi.NSOP_PX] * 4 + [_abi.NSOP_SYRK, _abi.NSOP_POLY,
                                                                  _abi.NSOP_PX_APPLY]
    assert kinds(std) == chain
    if gram:
        assert kinds(ops).count(_abi.NSOP_SYMM) == 9 and kinds(ops).count(_abi.NSOP_SYRK) == 2
        assert kinds(ops).count(_abi.NSOP_POLY) == 5 and kinds(ops)[-1] == _abi.NSOP_PX_APPLY
    else:
        assert kinds(ops) == chain
    # fp32 Newton-Schulz and other iteration counts keep the chain
    assert kinds(_abi.ns_plan(rows, cols, _abi.F32, 5)) == chain
    assert _abi.NSOP_SYMM not in kinds(_abi.ns_plan(rows, cols, _abi.BF16, 4))
    # NO_APPLY: the same launches, the last one writing an X stack
    na = _abi.ns_plan(rows, cols, _abi.BF16, 5, _abi.NS_NO_APPLY)
    assert kinds(na)[:-1] == kinds(ops)[:-1] and na[-1].kind == _abi.NSOP_PX
    assert (na[-1].in0, na[-1].in1) == (ops[-1].in0, ops[-1].in1)
    assert _abi.ns_output_buffer(rows, cols, _abi.BF16, 5) == na[-1].out


def _block(m, n, seed, spectrum=None):
    gen = torch.Generator().manual_seed(seed)
    if spectrum is None:
        return torch.randn(m, n, generator=gen, dtype=torch.float64) * 1e-3
    u, _ = torch.linalg.qr(torch.randn(m, m, generator=gen, dtype=torch.float64))
    v, _ = torch.linalg.qr(torch.randn(n, m, generator=gen, dtype=torch.float64))
    return (u * spectrum) @ v.T


@pytest.mark.parametrize("flags", [0, _abi.NS_STANDARD])
@pytest.mark.parametrize("rows,cols", [(1024, 2752), (512, 1376), (1024, 1024)])
def test_plan_equals_newton_schulz_in_fp64(rows, cols, flags):
    """Every plan (the op list depends only on eligibility, so it runs here on a
    smaller block of the same kind) reproduces fp64 Newton-Schulz."""
    ops = _abi.ns_plan(rows, cols, _abi.BF16, 5, flags | _abi.NS_NO_APPLY)
    m, n = (48, 136) if rows != cols else (48, 48)
    for seed in range(3):
        x = _block(m, n, seed)
        got = run_plan(ops, x)
        truth = ns_fp64(x[None])[0]
        assert float(rel_fro(got[None], truth[None])) < 1e-10
    # the apply plan's update is the same X
    apply_ops = _abi.ns_plan(rows, cols, _abi.BF16, 5, flags)
    x = _block(m, n, 5)
    assert torch.allclose(run_plan(apply_ops, x), ns_fp64(x[None])[0], rtol=0, atol=1e-12)


def test_gram_plan_within_the_bar_in_bf16_on_ill_conditioned_blocks():
    m, n = 256, 688
    ops = _abi.ns_plan(n, m, _abi.BF16, 5, _abi.NS_NO_APPLY)   # tall block: Newton-Schulz on the transpose
    assert _abi.NSOP_SYMM in kinds(ops)
    d = torch.float64
    spectra = [None, torch.logspace(0, -3, m, dtype=d), torch.logspace(0, -5, m, dtype=d),
               torch.cat([torch.logspace(0, -1, 16, dtype=d), torch.full((m - 16,), 1e-3, dtype=d)]),
               torch.cat([torch.ones(1, dtype=d), torch.full((m - 1,), 1e-4, dtype=d)])]
    for i, sv in enumerate(spectra):
        x = bf16(_block(m, n, 10 + i, sv))
        truth = ns_fp64(x[None])[0]
        ref = newton_schulz_batched(x[None].to(torch.bfloat16))[0].double()
        e_ref = float(rel_fro(ref[None], truth[None]))
        e_gram = float(rel_fro(run_plan(ops, x, bf16)[None], truth[None]))
        assert e_gram <= 1.5 * e_ref + 2e-3, (i, e_gram, e_ref)
    # the Gram recursion without the rebuild of X (a plan of the same ops with
    # the restart's PX and SYRK removed) drifts past the bar on the last two
    x = bf16(_block(m, n, 14, spectra[4]))
    truth = ns_fp64(x[None])[0]
    e_ref = float(rel_fro(newton_schulz_batched(x[None].to(torch.bfloat16))[0].double()[None], truth[None]))
    assert float(rel_fro(_gram_no_restart(x, bf16)[None], truth[None])) > 1.5 * e_ref + 2e-3


def _gram_no_restart(x0, rnd):
    """Five Gram iterations from A_0 = s^2 X X^T with no rebuild of X."""
    m = x0.shape[0]
    s = 1.0 / (float(torch.linalg.matrix_norm(x0)) + NS_EPS)
    eye = torch.eye(m, dtype=x0.dtype)
    a = rnd(s * s * (x0 @ x0.T))
    q = None
    for k in range(5):
        p = rnd(A_C * eye + B_C * a + C_C * (a @ a))
        q = p if q is None else rnd(p @ q)
        if k < 4:
            a = rnd(p @ rnd(p @ a))
    return rnd(s * (q @ x0))


def test_optimizer_ns_form_selects_the_plan_flags():
    """``ns_form`` maps to the plan flags; anything else is rejected at
    construction (no GPU call)."""
    from monarch_muon_amd import MonarchMuonOptimizer
    p = torch.zeros(2, 8, 8, requires_grad=True)
    assert MonarchMuonOptimizer([p], [])._ns_flags == 0
    assert MonarchMuonOptimizer([p], [], ns_form="standard")._ns_flags == _abi.NS_STANDARD
    with pytest.raises(ValueError):
        MonarchMuonOptimizer([p], [], ns_form="gram")


def test_plan_entry_point_validates_its_arguments():
    """mmuon_ns_plan: the op count with a NULL array, MMUON_ERANGE when the
    array is too short, MMUON_EINVAL for a bad iteration count, shape or dtype
    (host-only calls)."""
    import ctypes as C
    lib = _abi.lib()
    n = lib.mmuon_ns_plan(1024, 2752, _abi.BF16, 5, 0, None, 0)
    assert n == 18
    short = (_abi.NsOp * 4)()
    assert lib.mmuon_ns_plan(1024, 2752, _abi.BF16, 5, 0, short, 4) == -3
    for args in [(1024, 2752, _abi.BF16, 0), (1024, 2752, _abi.BF16, 65), (0, 2752, _abi.BF16, 5),
                 (1024, 2752, 7, 5)]:
        assert lib.mmuon_ns_plan(*args, 0, None, 0) == -1, args
    assert lib.mmuon_ns_plan(1024, 1024, _abi.F32, 5, 0, None, 0) == 15
