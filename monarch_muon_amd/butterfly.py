"""Monarch butterfly multiply on the MI355X kernels (``mmuon_butterfly_fwd`` / ``_bwd``).

The same interface as the reference's opaque custom ops
(pretrain/src/models/monarch/monarch_ops.py:23-114):

* ``butterfly_blk_op(x2, w1, w2) -> (out_blk, out1)``: ``x2`` (B, k p), ``w1`` (k, q, p),
  ``w2`` (l, s, r); ``out_blk`` (B, l, s) is the blocked output, ``out1`` (l, B, r) the riffled
  intermediate saved for the backward (monarch_ops.py:41-46).
* ``butterfly_blk_bwd_op(x2, w1, w2, out1, dout_blk) -> (dx, dw1, dw2)`` (monarch_ops.py:57-82).
* ``butterfly_blk(x, w1, w2)``: the differentiable wrapper with the reference's autocast cast and
  feature-order interleave (monarch_ops.py:105-114).

Both ops are registered with ``torch.library`` (namespace ``mmuon``) with fake implementations,
so ``torch.compile`` keeps them opaque as the reference's do.  The riffle between the two
products and its inverse in the backward are folded into the kernels' addressing; no
permutation pass runs.  bf16 only (the reference runs these products under bf16 autocast); the
kernels need p, q, s multiples of 8 and q / nblocks a multiple of 32, which every Monarch layer of
the reference's models satisfies.  Other inputs raise; there is no fallback.
"""
from __future__ import annotations

import ctypes as C

import torch

from . import _abi

__all__ = ["butterfly_blk", "butterfly_blk_op", "butterfly_blk_bwd_op", "patch_monarch_linear"]


def _args(x2: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> _abi.ButterflyArgs:
    _abi._require_cuda(x2, w1, w2)
    for name, t in (("x", x2), ("w1", w1), ("w2", w2)):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"the MI355X butterfly computes in bfloat16; {name} is {t.dtype} "
                            "(run under torch.autocast(dtype=torch.bfloat16) or pass bf16 tensors)")
    if w1.dim() != 3 or w2.dim() != 3 or x2.dim() != 2:
        raise ValueError("expected x2 (B, n), w1 (k, q, p), w2 (l, s, r)")
    k, q, p = w1.shape
    l, s, r = w2.shape
    if k != l or q != r or x2.shape[1] != k * p:
        raise ValueError(f"butterfly shapes do not chain: x2 {tuple(x2.shape)}, w1 {tuple(w1.shape)}, "
                         f"w2 {tuple(w2.shape)} (need k == l, q == r, n == k p)")
    a = _abi.ButterflyArgs()
    a.tokens, a.nblocks, a.q, a.p, a.s, a.dtype = x2.shape[0], k, q, p, s, _abi.BF16
    a.x, a.w1, a.w2 = x2.data_ptr(), w1.data_ptr(), w2.data_ptr()
    return a


def _fwd(x2: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    x2, w1, w2 = x2.contiguous(), w1.contiguous(), w2.contiguous()
    a = _args(x2, w1, w2)
    B = x2.shape[0]
    l, s, r = w2.shape
    out_blk = torch.empty(B, l, s, device=x2.device, dtype=x2.dtype)
    out1 = torch.empty(l, B, r, device=x2.device, dtype=x2.dtype)
    a.out, a.out1 = out_blk.data_ptr(), out1.data_ptr()
    _abi.check(_abi.lib().mmuon_butterfly_fwd(C.byref(a), _abi.stream_handle(x2.device)), "mmuon_butterfly_fwd")
    return out_blk, out1


def _bwd(x2, w1, w2, out1, dout_blk):
    x2, w1, w2 = x2.contiguous(), w1.contiguous(), w2.contiguous()
    out1, dout_blk = out1.contiguous(), dout_blk.contiguous()
    a = _args(x2, w1, w2)
    B = x2.shape[0]
    l, s, r = w2.shape
    if tuple(out1.shape) != (l, B, r) or tuple(dout_blk.shape) != (B, l, s):
        raise ValueError(f"out1 {tuple(out1.shape)} / dout {tuple(dout_blk.shape)} do not match the forward")
    if out1.dtype != torch.bfloat16 or dout_blk.dtype != torch.bfloat16:
        raise TypeError("out1 and dout must be bfloat16")
    _abi._require_cuda(out1, dout_blk)
    dx = torch.empty_like(x2)
    dw1 = torch.empty_like(w1)
    dw2 = torch.empty_like(w2)
    a.out1, a.dout, a.dx, a.dw1, a.dw2 = (out1.data_ptr(), dout_blk.data_ptr(), dx.data_ptr(),
                                          dw1.data_ptr(), dw2.data_ptr())
    nbytes = _abi.lib().mmuon_butterfly_workspace(C.byref(a))
    ws = torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=x2.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _abi.check(_abi.lib().mmuon_butterfly_bwd(C.byref(a), _abi.stream_handle(x2.device)), "mmuon_butterfly_bwd")
    return dx, dw1, dw2


@torch.library.custom_op("mmuon::butterfly_blk", mutates_args=())
def butterfly_blk_op(x2: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    return _fwd(x2, w1, w2)


@butterfly_blk_op.register_fake
def _(x2, w1, w2):
    B = x2.shape[0]
    l, s, r = w2.shape
    return x2.new_empty(B, l, s), x2.new_empty(l, B, r)


@torch.library.custom_op("mmuon::butterfly_blk_bwd", mutates_args=())
def butterfly_blk_bwd_op(x2: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor, out1: torch.Tensor,
                         dout_blk: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _bwd(x2, w1, w2, out1, dout_blk)


@butterfly_blk_bwd_op.register_fake
def _(x2, w1, w2, out1, dout_blk):
    return x2.new_empty(x2.shape), w1.new_empty(w1.shape), w2.new_empty(w2.shape)


def _setup_context(ctx, inputs, output):
    x2, w1, w2 = inputs
    ctx.save_for_backward(x2, w1, w2, output[1])


def _backward(ctx, dout_blk, dout1_unused):
    x2, w1, w2, out1 = ctx.saved_tensors
    return butterfly_blk_bwd_op(x2, w1, w2, out1, dout_blk.contiguous())


butterfly_blk_op.register_autograd(_backward, setup_context=_setup_context)


def butterfly_blk(x: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """``x`` (..., k p) -> (..., s l) in the layer's feature order (monarch_ops.py:105-114)."""
    if torch.is_autocast_enabled():
        dt = torch.get_autocast_dtype("cuda")
        x, w1, w2 = x.to(dt), w1.to(dt), w2.to(dt)
    batch_shape, n = x.shape[:-1], x.shape[-1]
    out_blk, _ = butterfly_blk_op(x.reshape(-1, n), w1, w2)
    B, l, s = out_blk.shape
    return out_blk.transpose(1, 2).reshape(*batch_shape, s * l)


def patch_monarch_linear(cls) -> None:
    """Route a ``MonarchLinear`` class's ``forward_matmul`` through the MI355X op (the reference's
    own switch, membench/src/models/monarch/monarch_ops.py:121-127, with this op)."""

    def forward_matmul(self, x):
        return self.postprocess(butterfly_blk(self.preprocess(x), self.blkdiag1, self.blkdiag2))

    cls.forward_matmul = forward_matmul
