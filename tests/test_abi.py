"""The C-ABI library: loads, exports every declared symbol, ctypes layouts match
the header, argument validation works (no GPU calls)."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

from monarch_muon_amd import _abi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mmuon.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mmuon_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _abi.lib()
    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_abi.SIGNATURES), "ctypes signature table out of sync with mmuon.h"


def test_struct_layouts_match_header(tmp_path):
    structs = {"mmuon_block_ref": _abi.BlockRef, "mmuon_block_fp8": _abi.BlockFp8,
               "mmuon_ns_layout_t": _abi.NsLayout, "mmuon_group": _abi.Group,
               "mmuon_adamw_tensor": _abi.AdamWTensor, "mmuon_adamw_args": _abi.AdamWArgs,
               "mmuon_adamw_fp8_tensor": _abi.AdamWFp8Tensor, "mmuon_grad_tensor": _abi.GradTensor,
               "mmuon_grad_norm_args": _abi.GradNormArgs, "mmuon_butterfly_args": _abi.ButterflyArgs,
               "mmuon_ns_op": _abi.NsOp}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} size %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname}.{fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split("\n")
    got = dict(l.rsplit(" ", 1) for l in out if l)
    for cname, py in structs.items():
        assert int(got[f"{cname} size"]) == C.sizeof(py), cname
        for fname, _ in py._fields_:
            assert int(got[f"{cname}.{fname}"]) == getattr(py, fname).offset, f"{cname}.{fname}"


def test_layout_geometry():
    lay = _abi.ns_layout(2752, 1024, _abi.BF16, 256)
    assert (lay.m, lay.n) == (1024, 2752)
    assert lay.mp % 256 == 0 and lay.np_ % 256 == 0 and lay.np_ >= 2752
    assert lay.x_bytes == 256 * lay.mp * lay.np_ * 2
    assert lay.a_bytes == 256 * lay.mp * lay.mp * 2
    lay = _abi.ns_layout(256, 688, _abi.F32, 4)
    assert (lay.m, lay.n, lay.mp) == (256, 688, 256) and lay.np_ % 64 == 0


@pytest.mark.parametrize("args", [(0, 4, _abi.BF16, 1), (4, 4, 7, 1), (4, 4, _abi.BF16, 0)])
def test_layout_rejects_bad_arguments(args):
    with pytest.raises(RuntimeError, match="mmuon_ns_layout failed"):
        _abi.ns_layout(*args)


def test_entry_points_reject_null_descriptors():
    lib = _abi.lib()
    assert lib.mmuon_momentum_pack(None, 0.9, None) == -1
    assert b"null group" in lib.mmuon_last_error()
    assert lib.mmuon_newton_schulz_apply(None, 5, None, 0.0, 0, None) == -1
    assert lib.mmuon_adamw(None, None) == -1
    g = _abi.Group(rows=64, cols=64, nblocks=1, param_dtype=_abi.BF16, grad_dtype=_abi.BF16,
                   buf_dtype=_abi.F32, ns_dtype=_abi.BF16, blocks=None)
    assert lib.mmuon_momentum_pack(C.byref(g), 0.9, None) == -1
    assert b"block table" in lib.mmuon_last_error()
    g.blocks = 16
    g.ns_dtype = 9
    assert lib.mmuon_momentum_pack(C.byref(g), 0.9, None) == -1
    assert b"ns_dtype" in lib.mmuon_last_error()


def test_product_path_refuses_cpu_tensors():
    import torch
    from monarch_muon_amd import MonarchMuonOptimizer
    p = torch.zeros(1, 8, 8, requires_grad=True)
    p.grad = torch.zeros_like(p)
    opt = MonarchMuonOptimizer([p], [])
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        opt.step()


def test_butterfly_entry_points_validate_before_launching():
    """Every descriptor here is invalid, so no kernel is launched (no GPU needed)."""
    lib = _abi.lib()
    a = _abi.ButterflyArgs(tokens=16, nblocks=4, q=64, p=64, s=64, dtype=_abi.BF16,
                           x=4096, w1=8192, w2=12288, out=16384, out1=20480)
    assert lib.mmuon_butterfly_fwd(None, None) == -1
    assert lib.mmuon_butterfly_fwd(C.byref(a), None) == -1           # q / nblocks = 16
    assert b"multiple of 32" in lib.mmuon_last_error()
    a.q, a.dtype = 128, _abi.F32
    assert lib.mmuon_butterfly_fwd(C.byref(a), None) == -1
    assert b"MMUON_BF16" in lib.mmuon_last_error()
    a.dtype, a.nblocks = _abi.BF16, 3
    assert lib.mmuon_butterfly_fwd(C.byref(a), None) == -1
    assert b"nblocks" in lib.mmuon_last_error()
    a.nblocks, a.p = 4, 60
    assert lib.mmuon_butterfly_fwd(C.byref(a), None) == -1
    assert b"multiples of 8" in lib.mmuon_last_error()
    a.p, a.x = 64, 4100
    assert lib.mmuon_butterfly_fwd(C.byref(a), None) == -1
    assert b"unaligned" in lib.mmuon_last_error()
    a.x, a.tokens = 4096, 1 << 24
    assert lib.mmuon_butterfly_fwd(C.byref(a), None) == -3
    a.tokens = 16
    # backward: dout, dx, dw1, dw2 present, workspace too small
    a.dout, a.dx, a.dw1, a.dw2, a.workspace, a.workspace_bytes = 24576, 28672, 32768, 36864, 40960, 16
    need = lib.mmuon_butterfly_workspace(C.byref(a))
    assert need >= 4 * 16 * 128 * 2
    assert lib.mmuon_butterfly_bwd(C.byref(a), None) == -1
    assert b"workspace" in lib.mmuon_last_error()


def test_hbm_probe_validates_before_launching():
    """The bench-only HBM probe (bench_probe.so, apart from libmmuon.so) rejects
    every malformed request before it launches (no GPU needed); libmmuon.so
    does not export it."""
    import bench_studies
    lib = bench_studies.probe_lib()
    assert not hasattr(_abi.lib(), "mmuon_hbm_stream")
    n = 1 << 20
    assert lib.probe_hbm_stream(8, 4096, 4096, n, 0, 16, None) == -1
    assert b"kind" in lib.probe_last_error()
    assert lib.probe_hbm_stream(2, 4096, 4096, n + 16, 0, 16, None) == -1   # not a multiple of 32
    assert b"multiple of 32" in lib.probe_last_error()
    assert lib.probe_hbm_stream(5, 4096, 4096, n, 0, 0, None) == -1
    assert b"grid" in lib.probe_last_error()
    for kind in (1, 2, 4, 5, 6, 7):      # every kind but the read probes needs dst
        assert lib.probe_hbm_stream(kind, None, 4096, n, 0, 16, None) == -1
        assert b"null" in lib.probe_last_error()
    for kind in (0, 2, 3, 5, 7):         # these read (kind 7 also writes) src
        assert lib.probe_hbm_stream(kind, 4096, None, n, 0, 16, None) == -1
    assert lib.probe_hbm_stream(6, 4100, 4096, n, 0, 16, None) == -1        # unaligned
    assert b"aligned" in lib.probe_last_error()
    # the read probes' guard store needs grid * 4096 (grid-stride) / grid * 16384 (spans) bytes of dst
    assert lib.probe_hbm_stream(0, 4096, 4096, 4096 * 64, 0, 65, None) == -1
    assert lib.probe_hbm_stream(3, 4096, 4096, 16384 * 16, 0, 17, None) == -1
    assert b"read probe" in lib.probe_last_error()
