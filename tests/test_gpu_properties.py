"""Exact properties of the momentum + Newton-Schulz path at the headline size
(6.89B-dense-reference model, nb=4: all 1408 + 256 + 128 blocks), checked on
every block, bit for bit, with no oracle computation:

- scale invariance: gradients and momentum doubled give the same Newton-Schulz
  output.  Every quantity on the way scales by a power of two -- the momentum
  update (buf * mu, + g), X = bf16(buf), the sums of squares (x4), the norm and
  its two bf16 roundings (x2), s = 1/norm (/2) -- and the Gram product takes
  s^2 and the first X update s, so the doubling cancels exactly.  A mistake in
  that fold (s for s^2, the scale applied twice or on another iteration, a norm
  over the wrong extent) breaks it.
- order invariance: the parameters in reverse order give every block the same
  Newton-Schulz output: a block's result depends neither on its position in the
  stacks nor on which workgroup or XCD computes it.

The step runs without the apply (NS_NO_APPLY), so the outputs stay in the
workspace X stacks, which are compared raw (panel layout, padding included).
"""
import ctypes as C

import pytest
import torch

from monarch_muon_amd import _abi
from monarch_muon_amd.plan import NS_COEFFS, MuonPlanner
from monarch_muon_amd.workloads import WORKLOADS, parameter_inventory

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
MU = 0.95


def _draw():
    w = WORKLOADS["6.89b-nb4"]
    gen = torch.Generator(device=DEV).manual_seed(5)
    params, grads, bufs = [], [], []
    for _, shape, is_muon in parameter_inventory(w):
        if not is_muon:
            continue
        params.append((torch.randn(shape, generator=gen, device=DEV) * 0.02).bfloat16())
        grads.append((torch.randn(shape, generator=gen, device=DEV) * 1e-3).bfloat16())
        bufs.append(torch.randn(shape, generator=gen, device=DEV) * 1e-3)
    return params, grads, bufs


def _ns_outputs(params, grads, bufs):
    """Run pack + Newton-Schulz (no apply) through the C ABI; per group: (member
    parameter indices, raw bf16 output stack [N, mp*np], a copy)."""
    planner = MuonPlanner()
    launches = planner.plan(params, grads, bufs, torch.bfloat16)
    lib, stream = _abi.lib(), _abi.stream_handle(DEV)
    coeffs = (C.c_float * 3)(*NS_COEFFS)
    out = {}
    for gl in launches:
        _abi.check(lib.mmuon_momentum_pack(C.byref(gl.struct), MU, stream), "pack")
        _abi.check(lib.mmuon_newton_schulz_apply(C.byref(gl.struct), 5, coeffs, 0.0, _abi.NS_NO_APPLY, stream), "ns")
        lay = gl.ws.layout
        per = lay.mp * lay.np_
        xs = gl.ws.x1 if _abi.ns_output_buffer(gl.rows, gl.cols, lay.ns_dtype, 5) == _abi.NSB_X1 else gl.ws.x0
        stack = xs.view(torch.bfloat16)[: gl.nblocks * per].view(gl.nblocks, per)
        out[(gl.rows, gl.cols)] = (list(gl.members), stack.clone())
    torch.cuda.synchronize()
    planner.release()
    return out


def test_doubled_gradients_and_momentum_give_the_same_newton_schulz_output():
    params, grads, bufs = _draw()
    base = _ns_outputs(params, grads, [b.clone() for b in bufs])
    doubled = _ns_outputs(params, [g * 2 for g in grads], [b * 2 for b in bufs])
    assert sorted(base) == [(1024, 1024), (1024, 2752), (2752, 1024)]
    for key in base:
        assert base[key][0] == doubled[key][0]
        a, b = base[key][1], doubled[key][1]
        assert bool(torch.isfinite(a.float()).all())
        assert torch.equal(a, b), f"group {key}: doubling the inputs changed the Newton-Schulz output"


def test_reversed_parameter_order_gives_every_block_the_same_output():
    params, grads, bufs = _draw()
    fwd = _ns_outputs(params, grads, [b.clone() for b in bufs])
    n = len(params)
    rev = _ns_outputs(params[::-1], grads[::-1], [b.clone() for b in bufs[::-1]])
    assert sorted(fwd) == sorted(rev)
    for key, (members, stack) in fwd.items():
        rmembers, rstack = rev[key]
        assert sorted(members) == sorted(n - 1 - i for i in rmembers)
        # block position of (parameter, block) in each stack
        nb = params[members[0]].shape[0]
        pos = {(i, k): j * nb + k for j, i in enumerate(members) for k in range(nb)}
        rpos = [pos[(n - 1 - i, k)] for i in rmembers for k in range(nb)]
        perm = torch.tensor(rpos, device=DEV)
        assert torch.equal(stack[perm], rstack), f"group {key}: a block's output depends on the parameter order"
