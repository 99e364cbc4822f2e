"""GPU parity of each Newton-Schulz stage on its own, through mmuon_ns_stage.

Every stage output is compared with an fp64 product of the stage's own bf16
inputs as the library left them in the workspace, so a stage is checked in
isolation (the end-to-end chain is covered in test_gpu_parity.py):

  SYRK  A  = s^2 X X^T          (tiles on and above the diagonal are stored)
  POLY  P  = a I + b A + c A A  (A's lower tiles are the transposes of its upper ones;
                                 a only on the diagonal of the m valid rows)
  PX    X' = s P X
  SYMM  C  = S1 S2              (two symmetric stacks; upper tiles stored; run through
                                 mmuon_ns_run_op into the sub-stacks of x1, on the
                                 shapes whose X stack holds two m x m stacks)

Bar: |stage - fp64| <= 2^-8 * max|fp64| per block (one bf16 step at the largest
entry; bf16 output rounding is at most half of that).  Diagonal 256 x 256 tiles
of A and P are stored in full and must be exactly symmetric.  The shapes cover
m = 1024 (four diagonal tiles per block, whose 32 x 32 MFMA tiles the kernels
deal over the waves), tall and wide blocks, and zero padding; the two largest
stacks have more tiles than the 256 persistent workgroups, so a workgroup runs
several tiles in a row (diagonal and upper tiles, tiles of different blocks)
through the same LDS ring and staging area.  The fp64 reference products run
on the GPU.
"""
import ctypes as C

import pytest
import torch

from monarch_muon_amd import _abi
from monarch_muon_amd.plan import NS_COEFFS, MuonPlanner

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TILE = 256
SHAPES = [(2, 1024, 1024), (1, 2752, 1024), (1, 1024, 2752), (3, 512, 512), (2, 96, 136), (2, 96, 600),
          (40, 1024, 1024), (30, 1024, 2752)]


def panels(t: torch.Tensor, nblocks: int, rows: int, cols: int) -> torch.Tensor:
    """A bf16 stack in 32-column panels ([N][cols/32][rows][32]) as row-major fp64 [N, rows, cols]."""
    v = t.view(torch.bfloat16)[: nblocks * rows * cols].view(nblocks, cols // 32, rows, 32)
    return v.permute(0, 2, 1, 3).reshape(nblocks, rows, cols).double()


def mirror_upper(a: torch.Tensor) -> torch.Tensor:
    """Full symmetric matrices from their stored 256 x 256 tiles on and above the diagonal."""
    n = a.shape[-1] // TILE
    out = a.clone()
    for ti in range(n):
        for tc in range(ti):
            out[:, ti * TILE:(ti + 1) * TILE, tc * TILE:(tc + 1) * TILE] = \
                a[:, tc * TILE:(tc + 1) * TILE, ti * TILE:(ti + 1) * TILE].transpose(1, 2)
    return out


def check_upper_tiles(got: torch.Tensor, ref: torch.Tensor, what: str) -> None:
    n = got.shape[-1] // TILE
    for b in range(got.shape[0]):
        bound = 2.0 ** -8 * float(ref[b].abs().max())
        for ti in range(n):
            for tc in range(ti, n):
                sl = (b, slice(ti * TILE, (ti + 1) * TILE), slice(tc * TILE, (tc + 1) * TILE))
                err = float((got[sl] - ref[sl]).abs().max())
                assert err <= bound, f"{what} block {b} tile ({ti},{tc}): max error {err:.3e} > {bound:.3e}"
            d = got[b, ti * TILE:(ti + 1) * TILE, ti * TILE:(ti + 1) * TILE]
            assert torch.equal(d, d.T), f"{what} block {b} diagonal tile {ti} is not exactly symmetric"


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_stage_outputs_against_fp64_products(shape):
    gen = torch.Generator().manual_seed(7)
    g = (torch.randn(shape, generator=gen) * 1e-3).to(DEV)
    p = torch.zeros_like(g, dtype=torch.bfloat16)
    buf = torch.zeros_like(g)
    (gl,) = MuonPlanner().plan([p], [g.bfloat16()], [buf], torch.bfloat16)
    lib, stream = _abi.lib(), _abi.stream_handle(DEV)
    coeffs = (C.c_float * 3)(*NS_COEFFS)
    a_c, b_c, c_c = NS_COEFFS
    lay, ws, nb = gl.ws.layout, gl.ws, gl.nblocks
    mp, np_ = lay.mp, lay.np_

    def stage(it, st):
        _abi.check(lib.mmuon_ns_stage(C.byref(gl.struct), it, 5, st, coeffs, C.c_float(0.0), _abi.NS_NO_APPLY,
                                      stream), "mmuon_ns_stage")
        torch.cuda.synchronize()

    _abi.check(lib.mmuon_momentum_pack(C.byref(gl.struct), 0.0, stream), "pack")  # X = bf16(g), s = 1/||X||
    torch.cuda.synchronize()
    s = ws.scale.double().view(nb, 1, 1)
    x = panels(ws.x0, nb, mp, np_)

    stage(0, 0)  # SYRK of the first iteration (scaled by s^2)
    a = panels(ws.a, nb, mp, mp)
    check_upper_tiles(a, s * s * (x @ x.transpose(1, 2)), "SYRK")

    stage(0, 1)  # POLY from the stored A
    full_a = mirror_upper(a)
    pm = panels(ws.p, nb, mp, mp)
    eye = torch.zeros(mp, mp, dtype=torch.float64, device=DEV)
    eye[range(lay.m), range(lay.m)] = 1.0
    check_upper_tiles(pm, a_c * eye + b_c * full_a + c_c * (full_a @ full_a), "POLY")
    # the padding rows and columns of P stay zero, its diagonal included
    assert float(pm[:, lay.m:, :].abs().max() if lay.m < mp else 0.0) == 0.0

    stage(0, 2)  # PX from the stored P and X (first iteration: scaled by s)
    full_p = mirror_upper(pm)
    ref = s * (full_p @ x)
    got = panels(ws.x1, nb, mp, np_)
    for b in range(nb):
        bound = 2.0 ** -8 * float(ref[b].abs().max())
        err = float((got[b] - ref[b]).abs().max())
        assert err <= bound, f"PX block {b}: max error {err:.3e} > {bound:.3e}"
    # the zero padding stays zero through every stage
    for pad in (got[:, lay.m:, :], got[:, :, lay.n:]):
        assert pad.numel() == 0 or float(pad.abs().max()) == 0.0

    if np_ < 2 * mp:
        return
    # SYMM (the Gram form's product of two commuting symmetric stacks): P A into
    # the first m x m sub-stack of x1, A P into the second (its offset: N mp^2)
    def run_op(kind, in0, in1, out):
        op = _abi.NsOp(kind, in0, in1, out, 0, 0)
        _abi.check(lib.mmuon_ns_run_op(C.byref(gl.struct), C.byref(op), coeffs, C.c_float(0.0), stream),
                   "mmuon_ns_run_op")
        torch.cuda.synchronize()

    run_op(_abi.NSOP_SYMM, _abi.NSB_P, _abi.NSB_A, _abi.NSB_X1_S0)
    run_op(_abi.NSOP_SYMM, _abi.NSB_A, _abi.NSB_P, _abi.NSB_X1_S1)
    sub = ws.x1.view(torch.bfloat16)[: 2 * nb * mp * mp]
    pa = panels(sub[: nb * mp * mp], nb, mp, mp)
    ap = panels(sub[nb * mp * mp:], nb, mp, mp)
    check_upper_tiles(pa, full_p @ full_a, "SYMM P A")
    check_upper_tiles(ap, full_a @ full_p, "SYMM A P")
    # zero padding of both operands gives zero padding, the diagonal included
    if lay.m < mp:
        assert float(pa[:, lay.m:, :].abs().max()) == 0.0 and float(ap[:, :, lay.m:].abs().max()) == 0.0


def test_run_op_rejects_invalid_ops():
    """mmuon_ns_run_op validates buffer kinds, overlaps and sub-stack room on the
    host before any launch."""
    g = torch.zeros(1, 256, 256, device=DEV)
    (gl,) = MuonPlanner().plan([torch.zeros_like(g, dtype=torch.bfloat16)], [g.bfloat16()], [g.clone()],
                               torch.bfloat16)
    lib, stream = _abi.lib(), _abi.stream_handle(DEV)
    coeffs = (C.c_float * 3)(*NS_COEFFS)
    bad = [(_abi.NSOP_SYMM, _abi.NSB_A, _abi.NSB_P, _abi.NSB_A),          # output is an operand
           (_abi.NSOP_SYMM, _abi.NSB_A, _abi.NSB_P, _abi.NSB_X1_S0),      # 256 x 256: no sub-stack room
           (_abi.NSOP_PX, _abi.NSB_P, _abi.NSB_X0, _abi.NSB_X0),          # PX in place
           (_abi.NSOP_SYRK, _abi.NSB_A, -1, _abi.NSB_P),                   # SYRK of a symmetric stack
           (9, _abi.NSB_A, _abi.NSB_P, _abi.NSB_X1)]
    for kind, i0, i1, o in bad:
        op = _abi.NsOp(kind, i0, i1, o, 0, 0)
        rc = lib.mmuon_ns_run_op(C.byref(gl.struct), C.byref(op), coeffs, C.c_float(0.0), stream)
        assert rc == -1, (kind, i0, i1, o, rc)


@pytest.mark.parametrize("shape", [(3, 1024, 2752), (2, 512, 512)], ids=lambda s: "x".join(map(str, s)))
def test_plan_ops_one_by_one_equal_newton_schulz_apply(shape):
    """The ops of ``mmuon_ns_plan`` run one at a time through
    ``mmuon_ns_run_op`` (how bench.py times each launch) give the bits of
    ``mmuon_newton_schulz_apply`` (Gram form and three-product chain)."""
    gen = torch.Generator().manual_seed(5)
    g = (torch.randn(shape, generator=gen) * 1e-3).to(DEV)
    outs = []
    for one_by_one in (False, True):
        p = torch.zeros_like(g, dtype=torch.bfloat16)
        (gl,) = MuonPlanner().plan([p], [g.bfloat16()], [torch.zeros_like(g)], torch.bfloat16)
        lib, stream = _abi.lib(), _abi.stream_handle(DEV)
        coeffs = (C.c_float * 3)(*NS_COEFFS)
        _abi.check(lib.mmuon_momentum_pack(C.byref(gl.struct), 0.0, stream), "pack")
        ops = _abi.ns_plan(gl.rows, gl.cols, _abi.BF16, 5, _abi.NS_NO_APPLY)
        if one_by_one:
            for op in ops:
                _abi.check(lib.mmuon_ns_run_op(C.byref(gl.struct), C.byref(op), coeffs, C.c_float(0.0), stream),
                           "mmuon_ns_run_op")
        else:
            _abi.check(lib.mmuon_newton_schulz_apply(C.byref(gl.struct), 5, coeffs, 0.0, _abi.NS_NO_APPLY, stream),
                       "mmuon_newton_schulz_apply")
        torch.cuda.synchronize()
        outs.append(gl.ws.x_view(ops[-1].out, torch.bfloat16, gl.nblocks).clone())
    assert torch.equal(outs[0], outs[1])
