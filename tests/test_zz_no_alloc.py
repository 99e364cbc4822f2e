"""``mmuon_grad_clip_coef_noalloc`` (no caller workspace: the partial sums and
norms live in the library's static per-GPU scratch array) against
``mmuon_grad_clip_coef`` (caller workspace), through the C ABI.

Both run the same kernels in the same order, so total norm and coefficient
must be bit-identical.  Two calls in a row, the second on a smaller input
(fewer chunks and tensors than the first left in the shared array), per
gradient dtype; and inputs beyond the array's size are rejected before any
launch.
"""
import ctypes as C

import pytest
import torch

from monarch_muon_amd import _abi
from monarch_muon_amd.plan import NORM_CHUNK, NormPlanner

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _args(nl, total, coef, max_norm, workspace):
    return _abi.GradNormArgs(tensors=nl.tensors.data_ptr(), chunks=nl.chunks.data_ptr(),
                             first_chunk=nl.first_chunk.data_ptr(), nchunks=nl.nchunks, ntensors=nl.ntensors,
                             chunk_elems=NORM_CHUNK, grad_dtype=_abi.dtype_code(nl.dtype), max_norm=max_norm,
                             partial=nl.partial.data_ptr() if workspace else None,
                             norms=nl.norms.data_ptr() if workspace else None,
                             total=total.data_ptr(), coef=coef.data_ptr())


def _grads(shapes, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return [(torch.randn(s, device=DEV, generator=g) * 1e-2).to(dtype) for s in shapes]


BIG = [(4, 1024, 1024), (4, 2752, 1024), (50304, 512), (4096,), (777,), (3, 256, 688)] * 3
SMALL = [(2, 256, 256), (300,), (64, 129)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_noalloc_clip_coef_equals_workspace_entry_point(dtype):
    lib = _abi.lib()
    stream = _abi.stream_handle(DEV)
    for call, (shapes, max_norm) in enumerate([(BIG, 1.0), (SMALL, 0.05)]):
        grads = _grads(shapes, dtype, seed=30 + call)
        nl = NormPlanner().plan(grads)
        assert nl.nchunks + nl.ntensors < _abi.NOALLOC_SCRATCH_FLOATS
        t_ws, c_ws = torch.full((1,), -1.0, device=DEV), torch.full((1,), -1.0, device=DEV)
        t_na, c_na = torch.full((1,), -2.0, device=DEV), torch.full((1,), -2.0, device=DEV)
        a = _args(nl, t_ws, c_ws, max_norm, workspace=True)
        _abi.check(lib.mmuon_grad_clip_coef(C.byref(a), stream), "mmuon_grad_clip_coef")
        b = _args(nl, t_na, c_na, max_norm, workspace=False)
        _abi.check(lib.mmuon_grad_clip_coef_noalloc(C.byref(b), stream), "mmuon_grad_clip_coef_noalloc")
        torch.cuda.synchronize()
        assert torch.equal(t_na, t_ws) and torch.equal(c_na, c_ws), (call, t_na, t_ws, c_na, c_ws)
        # and both are torch's clip_grad_norm_ total in the gradients' dtype
        ref = torch.linalg.vector_norm(torch.stack([torch.linalg.vector_norm(g.float()) for g in grads]))
        assert abs(float(t_na) - float(ref)) <= 1e-2 * float(ref), (float(t_na), float(ref))
        assert 0.0 < float(c_na) <= 1.0


def test_noalloc_rejects_inputs_beyond_the_scratch_array():
    lib = _abi.lib()
    grads = _grads(SMALL, torch.bfloat16, seed=40)
    nl = NormPlanner().plan(grads)
    total, coef = torch.zeros(1, device=DEV), torch.zeros(1, device=DEV)
    a = _args(nl, total, coef, 1.0, workspace=False)
    a.nchunks = _abi.NOALLOC_SCRATCH_FLOATS   # more partial sums than the array holds: rejected before launching
    rc = lib.mmuon_grad_clip_coef_noalloc(C.byref(a), _abi.stream_handle(DEV))
    assert rc == -3
    assert "scratch" in lib.mmuon_last_error().decode()
    torch.cuda.synchronize()
    assert float(total) == 0.0 and float(coef) == 0.0


def test_noalloc_clip_coef_under_graph_capture():
    """Captured into a HIP graph (after one call outside capture, which looks up
    the scratch array's device address) and replayed on new gradient values:
    every replay equals the workspace entry point run eagerly on the same
    values, with the program's own eager work and synchronisations between the
    replays."""
    lib = _abi.lib()
    grads = _grads(BIG[:6], torch.bfloat16, seed=50)
    nl = NormPlanner().plan(grads)
    t_na, c_na = torch.zeros(1, device=DEV), torch.zeros(1, device=DEV)
    t_ws, c_ws = torch.zeros(1, device=DEV), torch.zeros(1, device=DEV)
    b = _args(nl, t_na, c_na, 0.5, workspace=False)
    a = _args(nl, t_ws, c_ws, 0.5, workspace=True)
    _abi.check(lib.mmuon_grad_clip_coef_noalloc(C.byref(b), _abi.stream_handle(DEV)), "warm-up")
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _abi.check(lib.mmuon_grad_clip_coef_noalloc(C.byref(b), _abi.stream_handle(DEV)), "captured call")
    gen = torch.Generator(device=DEV).manual_seed(51)
    for replay in range(4):
        for g in grads:   # new values in the same tensors (the graph holds their addresses)
            g.copy_((torch.randn(g.shape, device=DEV, generator=gen) * 10.0 ** -(replay + 1)).to(g.dtype))
        t_na.fill_(-1.0)
        c_na.fill_(-1.0)
        torch.cuda.synchronize()
        graph.replay()
        _abi.check(lib.mmuon_grad_clip_coef(C.byref(a), _abi.stream_handle(DEV)), "eager workspace call")
        torch.cuda.synchronize()
        assert torch.equal(t_na, t_ws) and torch.equal(c_na, c_ws), (replay, t_na, t_ws, c_na, c_ws)
    del graph
