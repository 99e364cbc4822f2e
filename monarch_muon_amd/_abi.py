"""ctypes binding of ``libmmuon.so`` (the C ABI declared in ``include/mmuon.h``).

The library is loaded lazily on first use and must exist: there is no
fallback implementation, so a missing or unloadable library raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import torch

LIB_PATH = Path(os.environ.get("MMUON_LIB", Path(__file__).resolve().parent / "libmmuon.so"))

F32, BF16, F8E4M3, F8E5M2 = 0, 1, 2, 3
GROUP_ALIGNED16 = 1
NS_NO_APPLY = 1
NS_STANDARD = 2
NS_HOLD_LAST = 4
ABI_VERSION = 7
# Newton-Schulz plan ops (MMUON_NSOP_*) and buffers (MMUON_NSB_*)
NSOP_SYRK, NSOP_POLY, NSOP_PX, NSOP_PX_APPLY, NSOP_SYMM = 0, 1, 2, 3, 4
NSB_X0, NSB_X1, NSB_A, NSB_P, NSB_X0_S0, NSB_X0_S1, NSB_X1_S0, NSB_X1_S1, NSB_PARAM = range(9)
NOALLOC_SCRATCH_FLOATS = 1 << 20

_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float8_e4m3fn: F8E4M3, torch.float8_e5m2: F8E5M2}
FP8_DTYPES = (torch.float8_e4m3fn, torch.float8_e5m2)


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPES[dt]
    except KeyError:
        raise TypeError(f"libmmuon supports float32, bfloat16, float8_e4m3fn and float8_e5m2 tensors, "
                        f"not {dt}") from None


class BlockRef(C.Structure):
    _fields_ = [("param", C.c_void_p), ("grad", C.c_void_p), ("buf", C.c_void_p)]


class BlockFp8(C.Structure):
    _fields_ = [("scale", C.c_void_p), ("expand", C.c_void_p), ("sqrt_minmax", C.c_void_p)]


class NsLayout(C.Structure):
    _fields_ = [("m", C.c_int32), ("n", C.c_int32), ("mp", C.c_int32), ("np_", C.c_int32),
                ("nparts", C.c_int32), ("ns_dtype", C.c_int32),
                ("x_bytes", C.c_int64), ("a_bytes", C.c_int64), ("part_bytes", C.c_int64)]


class Group(C.Structure):
    _fields_ = [("rows", C.c_int32), ("cols", C.c_int32), ("nblocks", C.c_int32),
                ("param_dtype", C.c_int32), ("grad_dtype", C.c_int32), ("buf_dtype", C.c_int32),
                ("ns_dtype", C.c_int32), ("flags", C.c_int32),
                ("blocks", C.c_void_p), ("fp8", C.c_void_p),
                ("x0", C.c_void_p), ("x1", C.c_void_p), ("a", C.c_void_p), ("p", C.c_void_p),
                ("partial", C.c_void_p), ("scale", C.c_void_p), ("grad_scale", C.c_void_p)]


class NsOp(C.Structure):
    _fields_ = [("kind", C.c_int32), ("in0", C.c_int32), ("in1", C.c_int32), ("out", C.c_int32),
                ("scaled", C.c_int32), ("iteration", C.c_int32)]


class AdamWTensor(C.Structure):
    _fields_ = [("param", C.c_void_p), ("grad", C.c_void_p), ("exp_avg", C.c_void_p),
                ("exp_avg_sq", C.c_void_p), ("numel", C.c_int64)]


class AdamWArgs(C.Structure):
    _fields_ = [("tensors", C.c_void_p), ("chunks", C.c_void_p), ("nchunks", C.c_int64),
                ("chunk_elems", C.c_int32), ("param_dtype", C.c_int32), ("grad_dtype", C.c_int32),
                ("state_dtype", C.c_int32), ("apply_weight_decay", C.c_int32),
                ("wd_factor", C.c_float), ("beta1", C.c_float), ("beta2", C.c_float),
                ("one_minus_beta1", C.c_float), ("one_minus_beta2", C.c_float),
                ("sqrt_bc2", C.c_float), ("eps", C.c_float), ("neg_step_size", C.c_float),
                ("grad_scale", C.c_void_p)]


class AdamWFp8Tensor(C.Structure):
    _fields_ = [("scale_m", C.c_void_p), ("expand_m", C.c_void_p), ("sqrt_minmax_m", C.c_void_p),
                ("scale_v", C.c_void_p), ("expand_v", C.c_void_p), ("sqrt_minmax_v", C.c_void_p)]


class GradTensor(C.Structure):
    _fields_ = [("grad", C.c_void_p), ("numel", C.c_int64)]


class GradNormArgs(C.Structure):
    _fields_ = [("tensors", C.c_void_p), ("chunks", C.c_void_p), ("first_chunk", C.c_void_p),
                ("nchunks", C.c_int64), ("ntensors", C.c_int32), ("chunk_elems", C.c_int32),
                ("grad_dtype", C.c_int32), ("max_norm", C.c_float), ("partial", C.c_void_p),
                ("norms", C.c_void_p), ("total", C.c_void_p), ("coef", C.c_void_p)]


class ButterflyArgs(C.Structure):
    _fields_ = [("tokens", C.c_int64), ("nblocks", C.c_int32), ("q", C.c_int32), ("p", C.c_int32),
                ("s", C.c_int32), ("dtype", C.c_int32),
                ("x", C.c_void_p), ("w1", C.c_void_p), ("w2", C.c_void_p), ("out", C.c_void_p),
                ("out1", C.c_void_p), ("dout", C.c_void_p), ("dx", C.c_void_p), ("dw1", C.c_void_p),
                ("dw2", C.c_void_p), ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t)]


# name -> (restype, argtypes)
SIGNATURES = {
    "mmuon_abi_version": (C.c_int, []),
    "mmuon_last_error": (C.c_char_p, []),
    "mmuon_ns_layout": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.c_int64, C.POINTER(NsLayout)]),
    "mmuon_momentum_pack": (C.c_int, [C.POINTER(Group), C.c_float, C.c_void_p]),
    "mmuon_fp8_momentum_pack": (C.c_int, [C.POINTER(Group), C.c_float, C.c_int32, C.c_float, C.c_void_p]),
    "mmuon_newton_schulz_apply": (C.c_int, [C.POINTER(Group), C.c_int32, C.POINTER(C.c_float),
                                            C.c_float, C.c_int32, C.c_void_p]),
    "mmuon_ns_stage": (C.c_int, [C.POINTER(Group), C.c_int32, C.c_int32, C.c_int32, C.POINTER(C.c_float),
                                 C.c_float, C.c_int32, C.c_void_p]),
    "mmuon_ns_plan": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.POINTER(NsOp),
                                C.c_int32]),
    "mmuon_ns_run_op": (C.c_int, [C.POINTER(Group), C.POINTER(NsOp), C.POINTER(C.c_float), C.c_float,
                                  C.c_void_p]),
    "mmuon_adamw": (C.c_int, [C.POINTER(AdamWArgs), C.c_void_p]),
    "mmuon_adamw_fp8": (C.c_int, [C.POINTER(AdamWArgs), C.POINTER(AdamWFp8Tensor), C.c_int32, C.c_int32,
                                  C.c_float, C.c_void_p]),
    "mmuon_fp8_quantize": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_int64, C.c_int32, C.c_int32, C.c_float, C.c_void_p]),
    "mmuon_fp8_dequantize": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_int64, C.c_int32, C.c_int32, C.c_void_p]),
    "mmuon_grad_clip_coef": (C.c_int, [C.POINTER(GradNormArgs), C.c_void_p]),
    "mmuon_grad_clip_coef_noalloc": (C.c_int, [C.POINTER(GradNormArgs), C.c_void_p]),
    "mmuon_butterfly_fwd": (C.c_int, [C.POINTER(ButterflyArgs), C.c_void_p]),
    "mmuon_butterfly_bwd": (C.c_int, [C.POINTER(ButterflyArgs), C.c_void_p]),
    "mmuon_butterfly_workspace": (C.c_size_t, [C.POINTER(ButterflyArgs)]),
}

_lib = None


def lib() -> C.CDLL:
    """Load ``libmmuon.so`` once; raise if it is missing or has another ABI."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m monarch_muon_amd.build` "
                "(the MI355X kernels have no fallback)")
        handle = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.mmuon_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {handle.mmuon_abi_version()}, expected {ABI_VERSION}")
        _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().mmuon_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ns_layout(rows: int, cols: int, ns_dtype: int, nblocks: int) -> NsLayout:
    out = NsLayout()
    check(lib().mmuon_ns_layout(rows, cols, ns_dtype, nblocks, C.byref(out)), "mmuon_ns_layout")
    return out


def ns_plan(rows: int, cols: int, ns_dtype: int, iters: int, flags: int = 0) -> list[NsOp]:
    """The launch plan ``mmuon_newton_schulz_apply`` runs for a group of
    (rows x cols) blocks (host-only: no GPU needed)."""
    n = lib().mmuon_ns_plan(rows, cols, ns_dtype, iters, flags, None, 0)
    check(min(n, 0), "mmuon_ns_plan")
    ops = (NsOp * n)()
    check(min(lib().mmuon_ns_plan(rows, cols, ns_dtype, iters, flags, ops, n), 0), "mmuon_ns_plan")
    return list(ops)


def ns_output_buffer(rows: int, cols: int, ns_dtype: int, iters: int, flags: int = NS_NO_APPLY) -> int:
    """Workspace X stack (0: x0, 1: x1) holding the Newton-Schulz output of a
    ``MMUON_NS_NO_APPLY`` run: the output of the plan's last op."""
    out = ns_plan(rows, cols, ns_dtype, iters, flags | NS_NO_APPLY)[-1].out
    assert out in (NSB_X0, NSB_X1)
    return out


def fp8_quantize(value: torch.Tensor, codes: torch.Tensor, scale: torch.Tensor, expand: torch.Tensor,
                 sqrt_minmax: torch.Tensor, signed: bool, fmt: torch.dtype = torch.float8_e4m3fn,
                 expand_min: float = 16) -> None:
    """Stand-alone codec: fp32 ``value`` -> FP8 ``codes`` (``fmt``: float8_e4m3fn
    or float8_e5m2; a uint8 ``codes`` tensor holds the raw bytes) + per-128
    metadata (in place)."""
    _require_cuda(value, codes, scale, expand, sqrt_minmax)
    assert value.dtype == torch.float32 and value.is_contiguous()
    assert codes.dtype in (torch.uint8, fmt) and codes.is_contiguous() and codes.numel() == value.numel()
    groups = (value.numel() + 127) // 128
    for t in (scale, expand, sqrt_minmax):
        assert t.dtype == torch.float32 and t.numel() >= groups and t.is_contiguous()
    check(lib().mmuon_fp8_quantize(value.data_ptr(), codes.data_ptr(), scale.data_ptr(), expand.data_ptr(),
                                   sqrt_minmax.data_ptr(), value.numel(), int(signed), dtype_code(fmt),
                                   float(expand_min), stream_handle(value.device)), "mmuon_fp8_quantize")


def fp8_dequantize(codes: torch.Tensor, scale: torch.Tensor, expand: torch.Tensor,
                   sqrt_minmax: torch.Tensor, out: torch.Tensor, signed: bool,
                   fmt: torch.dtype = torch.float8_e4m3fn) -> None:
    _require_cuda(codes, scale, expand, sqrt_minmax, out)
    assert out.dtype == torch.float32 and out.is_contiguous() and codes.is_contiguous()
    assert codes.dtype in (torch.uint8, fmt) and out.numel() == codes.numel()
    check(lib().mmuon_fp8_dequantize(codes.data_ptr(), scale.data_ptr(), expand.data_ptr(),
                                     sqrt_minmax.data_ptr(), out.data_ptr(), out.numel(), int(signed),
                                     dtype_code(fmt), stream_handle(out.device)), "mmuon_fp8_dequantize")


def _require_cuda(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("libmmuon kernels need tensors on a ROCm GPU (no CPU path)")
