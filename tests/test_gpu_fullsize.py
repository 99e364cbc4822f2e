"""The headline workload at full size: every Monarch block of the 6.89B-dense-
reference model (nb=4; 1408 + 256 + 128 blocks, 2.56B elements, fp32
momentum), one step on the GPU.

Size-independent checks over the whole step:
- the momentum of every parameter equals torch's GPU ops on the same values
  (``buf * mu + g``, the reference's two foreach roundings), bit for bit;
- the Newton-Schulz output (the step run without the apply) of the first and
  the last block of every group -- the last 1024 x 1024 block sits 2.9 GB
  into its workspace stacks, beyond 2^31 bytes -- is within 1.5x the
  reference's own bf16 error of fp64 Newton-Schulz (+2e-3), as in the
  one-layer test;
- every block of every parameter (all 1792) equals, bit for bit, the
  reference's apply run by torch on the GPU: a foreach add of the Newton-Schulz
  output the library left in its workspace with alpha = -lr sqrt(rows/cols).
"""
import ctypes as C

import pytest
import torch

from monarch_muon_amd import MonarchMuonOptimizer, _abi
from monarch_muon_amd.plan import NS_COEFFS, MuonPlanner
from monarch_muon_amd.workloads import WORKLOADS, parameter_inventory
from oracle.step import newton_schulz_batched
from oracle.truth import ns_fp64, rel_fro

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
LR, MU = 0.02, 0.95


def _draw():
    w = WORKLOADS["6.89b-nb4"]
    gen = torch.Generator(device=DEV).manual_seed(3)
    params, bufs = [], []
    for _, shape, is_muon in parameter_inventory(w):
        if not is_muon:
            continue
        p = (torch.randn(shape, generator=gen, device=DEV) * 0.02).bfloat16()
        p.grad = (torch.randn(shape, generator=gen, device=DEV) * 1e-3).bfloat16()
        params.append(p)
        bufs.append(torch.randn(shape, generator=gen, device=DEV) * 1e-3)
    return params, bufs


def test_full_6p89b_step():
    params, bufs = _draw()
    w0 = [p.clone() for p in params]
    # torch's GPU foreach ops on the same values: the expected momentum
    ref_bufs = [b.clone() for b in bufs]
    torch._foreach_mul_(ref_bufs, MU)
    torch._foreach_add_(ref_bufs, [p.grad for p in params])

    # 1) the step without the apply, through the C ABI: Newton-Schulz outputs
    mom = [b.clone() for b in bufs]
    planner = MuonPlanner()
    launches = planner.plan(params, [p.grad for p in params], mom, torch.bfloat16)
    assert [(gl.rows, gl.cols, gl.nblocks) for gl in launches] == [(1024, 1024, 1408), (2752, 1024, 256),
                                                                   (1024, 2752, 128)]
    lib, stream = _abi.lib(), _abi.stream_handle(DEV)
    coeffs = (C.c_float * 3)(*NS_COEFFS)
    ns_out, stacks = {}, []
    for gl in launches:
        _abi.check(lib.mmuon_momentum_pack(C.byref(gl.struct), MU, stream), "pack")
        _abi.check(lib.mmuon_newton_schulz_apply(C.byref(gl.struct), 5, coeffs, 0.0, _abi.NS_NO_APPLY, stream), "ns")
        torch.cuda.synchronize()
        lay = gl.ws.layout
        # block order inside the group: member parameters in order, blocks in order
        owner = [(i, k) for i in gl.members for k in range(params[i].shape[0])]
        assert len(owner) == gl.nblocks
        x = gl.ws.x_view(_abi.ns_output_buffer(gl.rows, gl.cols, lay.ns_dtype, 5), torch.bfloat16, gl.nblocks)
        for blk in (0, gl.nblocks - 1):
            u = x[blk, :lay.m, :lay.n].float()
            ns_out[owner[blk]] = (u.t() if gl.transposed else u).contiguous()
        # the whole output stack in each parameter's orientation, for the apply check
        u = x[:, :lay.m, :lay.n]
        stacks.append((gl, (u.transpose(1, 2) if gl.transposed else u).contiguous()))
        del x, u
    for b, r in zip(mom, ref_bufs):
        assert torch.equal(b, r), "momentum must match torch's GPU ops bit for bit"
    del mom

    worst = {}
    for (i, k), ours in ns_out.items():
        src = ref_bufs[i][k:k + 1].cpu().to(torch.bfloat16)
        truth = ns_fp64(src.double())
        e_ours = float(rel_fro(ours.cpu()[None].double(), truth).max())
        e_ref = float(rel_fro(newton_schulz_batched(src).double(), truth).max())
        key = tuple(params[i].shape[1:])
        worst[key] = max(worst.get(key, 0.0), e_ours)
        assert e_ours <= 1.5 * e_ref + 2e-3, (key, i, k, e_ours, e_ref)
    print("full 6.89B step, sampled Newton-Schulz error vs fp64:", worst)

    # 2) the full optimizer step (with the apply) on the original values
    opt = MonarchMuonOptimizer(params, [], lr=LR, momentum=MU)
    for p, b in zip(params, bufs):
        opt.state[p]["momentum_buffer"] = b
    opt.step()
    torch.cuda.synchronize()
    for p, r in zip(params, ref_bufs):
        assert torch.equal(opt.state[p]["momentum_buffer"], r)
    checked = 0
    for gl, stack in stacks:
        alpha = -LR * (gl.rows / gl.cols) ** 0.5
        b0 = 0
        for i in gl.members:
            nb = params[i].shape[0]
            expect = [w0[i].clone()]
            # the reference's apply (membench monarch_muon.py:165-170) run by torch on the GPU
            torch._foreach_add_(expect, [stack[b0:b0 + nb]], alpha=alpha)
            assert torch.equal(params[i].data, expect[0]), i
            checked += nb
            b0 += nb
        assert b0 == gl.nblocks
    assert checked == 1792
    print(f"apply checked on all {checked} blocks: bit-identical to torch's foreach add on the GPU")
