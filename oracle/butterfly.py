"""torch-CPU restatement of the Monarch butterfly multiply and its backward -- test infrastructure.

Restates ``pretrain/src/models/monarch/monarch_ops.py`` (the membench copy is the same op):

* ``butterfly_fwd``  -- ``_butterfly_fwd_blocked`` (``:23-36``) with the eager riffle of ``:33-35``;
* ``butterfly_bwd``  -- ``_butterfly_blk_bwd_op`` (``:57-82``) with the eager unriffle of ``:75-78``;
* ``butterfly_blk``  -- the feature-order interleave of ``butterfly_blk`` (``:105-114``).

Each product is an fp32 (fp64 for fp64 inputs) batched matmul of the given values, rounded to the
input dtype, which is where the reference's bf16 ``bmm`` calls round (the reference runs them under
bf16 autocast).  The summation order inside one product is the BLAS's and is not pinned: the HIP
path is compared with a tolerance.

Pinning (``tests/test_oracle_butterfly.py``):

* ``monarch_dense`` builds the dense matrix of the layer from an index formula (one outer product
  per (plane, column) pair), independent of the reshape/permute chain.  The forward must equal
  ``x @ M^T`` and the backward the autograd of that dense product (fp64) -- the reference's own
  check of its forward (``projection/test_monarch_blocks.py:59-72``) plus its backward.
* ``riffle`` / ``unriffle`` against the index formulas the reference's Triton kernels state
  (``monarch_riffle.py:27-45`` and ``:63``: ``dout1[b, k, j*NBK+l] = dt[l, b, k*QSUB+j]``) and
  against the alternative riffle expression of ``projection/test_monarch_blocks.py:28``.
* The rank structure the reference's projection test asserts (``test_monarch_blocks.py:74-84``):
  rows with one residue mod nblocks and one input chunk form a block of rank <= q / nblocks.
"""
from __future__ import annotations

import torch


def _acc(dt: torch.dtype) -> torch.dtype:
    return torch.float64 if dt == torch.float64 else torch.float32


def riffle(out1: torch.Tensor, l: int) -> torch.Tensor:
    """``out1`` (k, B, q) -> ``t`` (l, B, r): ``t[ll, b, i] = out1 flat (b, i l + ll)`` (monarch_ops.py:33-35)."""
    k, B, q = out1.shape
    r = k * q // l
    return out1.transpose(0, 1).reshape(B, r, l).permute(2, 0, 1).contiguous()


def unriffle(dt: torch.Tensor, k: int, q: int) -> torch.Tensor:
    """``dt`` (l, B, r) -> ``dout1`` (k, B, q), the inverse of ``riffle`` (monarch_ops.py:75-78)."""
    l, B, r = dt.shape
    return dt.transpose(0, 1).transpose(-1, -2).contiguous().reshape(B, k, q).transpose(0, 1)


def butterfly_fwd(x2: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """``(out_blk (B, l, s), out1 (l, B, r))`` of ``_butterfly_fwd_blocked`` (monarch_ops.py:23-36)."""
    dt, acc = x2.dtype, _acc(x2.dtype)
    B = x2.shape[0]
    k, q, p = w1.shape
    l, s, r = w2.shape
    x_r = x2.to(acc).reshape(B, k, p).transpose(0, 1)
    out1 = torch.bmm(x_r, w1.to(acc).transpose(-1, -2).contiguous()).to(dt)       # (k, B, q)
    t = riffle(out1, l)                                                             # (l, B, r)
    out2 = torch.bmm(t.to(acc), w2.to(acc).transpose(-1, -2).contiguous()).to(dt)  # (l, B, s)
    return out2.transpose(0, 1).contiguous(), t


def butterfly_bwd(x2, w1, w2, out1, dout_blk):
    """``(dx, dw1, dw2)`` of ``_butterfly_blk_bwd_op`` (monarch_ops.py:57-82); ``out1`` is the riffled
    intermediate ``t`` saved by the forward, ``dout_blk`` the (B, l, s) blocked gradient."""
    dt, acc = x2.dtype, _acc(x2.dtype)
    B = x2.shape[0]
    k, q, p = w1.shape
    l, s, r = w2.shape
    dout = dout_blk.to(acc).permute(1, 0, 2)                                      # (l, B, s)
    dw2 = torch.bmm(dout.transpose(-1, -2), out1.to(acc)).to(dt)                  # (l, s, r)
    dt_ = torch.bmm(dout, w2.to(acc)).to(dt)                                      # (l, B, r)
    dout1 = unriffle(dt_, k, q).to(acc)                                           # (k, B, q)
    dx = torch.bmm(dout1, w1.to(acc)).transpose(0, 1).reshape(B, k * p).to(dt)
    x_r = x2.to(acc).reshape(B, k, p).transpose(0, 1)
    dw1 = torch.bmm(dout1.transpose(-1, -2), x_r).to(dt)                          # (k, q, p)
    return dx, dw1, dw2


def butterfly_blk(x2: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """(B, k p) -> (B, s l) in the layer's feature order: ``y[b, j l + ll] = out_blk[b, ll, j]``."""
    out_blk, _ = butterfly_fwd(x2, w1, w2)
    B, l, s = out_blk.shape
    return out_blk.transpose(1, 2).reshape(B, s * l)


def blocked_grad(dy: torch.Tensor, l: int) -> torch.Tensor:
    """Feature-order gradient (B, s l) -> the blocked (B, l, s) gradient the backward op receives."""
    B, n = dy.shape
    return dy.reshape(B, n // l, l).transpose(1, 2).contiguous()


def monarch_dense(w1: torch.Tensor, w2: torch.Tensor) -> torch.Tensor:
    """Dense (s l, k p) matrix of the layer, ``y = x M^T``, from the index formula

        M[j l + ll, kk p + c] = sum over i with (i l + ll) // q == kk of
                                w2[ll, j, i] * w1[kk, (i l + ll) % q, c],

    one outer product per (ll, i).  Differentiable in w1 and w2."""
    k, q, p = w1.shape
    l, s, r = w2.shape
    assert k * q == l * r
    M = torch.zeros(s * l, k * p, dtype=w1.dtype)
    for ll in range(l):
        rows = torch.arange(s) * l + ll
        for i in range(r):
            kk, jq = divmod(i * l + ll, q)
            M = M.index_add(0, rows, torch.nn.functional.pad(torch.outer(w2[ll, :, i], w1[kk, jq, :]),
                                                              (kk * p, (k - 1 - kk) * p)))
    return M
