"""Pins the butterfly oracle (oracle/butterfly.py) before it checks the HIP kernels.

The dense-matrix check is the reference's own check of its forward
(projection/test_monarch_blocks.py:59-72, its shape list, padded shapes
included); the backward is checked against autograd through that dense matrix,
the riffle against the index formulas the reference's Triton kernels state.  A
transposed factor, a riffle in the wrong direction or a swapped gradient fails
one of them.
"""
import pytest
import torch

from oracle import butterfly as bf
from oracle.shapes import monarch_factors

# (n_out, n_in, nblocks) of projection/test_monarch_blocks.py:60, plus the Monarch
# factors of the benchmark models at reduced width
SHAPES = [(64, 64, 4), (96, 48, 4), (48, 96, 4), (50, 70, 4), (70, 50, 8), (33, 130, 8),
          (128, 48, 2), (48, 128, 2)]


def factors(n_out, n_in, nb, seed=0, dtype=torch.float64):
    s1, s2 = monarch_factors(n_in, n_out, nb)
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*s1, generator=g, dtype=dtype), torch.randn(*s2, generator=g, dtype=dtype)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_forward_is_the_dense_monarch_product(shape):
    w1, w2 = factors(*shape)
    k, q, p = w1.shape
    x = torch.randn(5, k * p, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    M = bf.monarch_dense(w1, w2)
    torch.testing.assert_close(bf.butterfly_blk(x, w1, w2), x @ M.T, rtol=1e-12, atol=1e-12)
    # the identity's image is the dense matrix itself (the reference's monarch_dense definition)
    torch.testing.assert_close(bf.butterfly_blk(torch.eye(k * p, dtype=torch.float64), w1, w2), M.T,
                               rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("shape", SHAPES, ids=str)
def test_backward_is_autograd_of_the_dense_product(shape):
    w1, w2 = factors(*shape, seed=3)
    k, q, p = w1.shape
    l, s, r = w2.shape
    g = torch.Generator().manual_seed(4)
    x = torch.randn(6, k * p, dtype=torch.float64, generator=g)
    dy = torch.randn(6, s * l, dtype=torch.float64, generator=g)
    xa, w1a, w2a = (t.clone().requires_grad_() for t in (x, w1, w2))
    (xa @ bf.monarch_dense(w1a, w2a).T).backward(dy)
    _, out1 = bf.butterfly_fwd(x, w1, w2)
    dx, dw1, dw2 = bf.butterfly_bwd(x, w1, w2, out1, bf.blocked_grad(dy, l))
    torch.testing.assert_close(dx, xa.grad, rtol=1e-11, atol=1e-11)
    torch.testing.assert_close(dw1, w1a.grad, rtol=1e-11, atol=1e-11)
    torch.testing.assert_close(dw2, w2a.grad, rtol=1e-11, atol=1e-11)


@pytest.mark.parametrize("l,q,B", [(2, 16, 3), (4, 32, 5), (4, 24, 2)])
def test_riffle_matches_the_stated_index_formulas(l, q, B):
    k = l
    out1 = torch.randn(k, B, q, generator=torch.Generator().manual_seed(5))
    t = bf.riffle(out1, l)
    qs = q // l
    # monarch_riffle.py:14-45: T[m, b, k*QSUB + j] = O1[b, k, j*NBK + m]
    for m in range(l):
        for kk in range(k):
            for j in range(qs):
                assert torch.equal(t[m, :, kk * qs + j], out1[kk, :, j * l + m])
    # projection/test_monarch_blocks.py:28, written with transpose(-1, -2) instead of permute
    r = k * q // l
    alt = out1.transpose(0, 1).reshape(B, r, l).transpose(-1, -2).contiguous().transpose(0, 1)
    assert torch.equal(t, alt)
    # monarch_riffle.py:63: dout1[b, k, j*NBK + l] = dt[l, b, k*QSUB + j]; unriffle inverts riffle
    d1 = bf.unriffle(t, k, q)
    assert torch.equal(d1, out1)
    for m in range(l):
        for kk in range(k):
            for j in range(qs):
                assert torch.equal(d1[kk, :, j * l + m], t[m, :, kk * qs + j])


@pytest.mark.parametrize("shape", [(64, 64, 2), (64, 64, 4), (64, 64, 8), (128, 32, 4), (32, 128, 4), (96, 48, 4)],
                         ids=str)
def test_dense_matrix_has_the_monarch_rank_structure(shape):
    """projection/test_monarch_blocks.py:74-84: rows with one residue mod nblocks and one
    contiguous input chunk form a block of rank q / nblocks, q = min(in_blk, out_blk)."""
    n_out, n_in, nb = shape
    w1, w2 = factors(*shape, seed=nb)
    M = bf.monarch_dense(w1, w2)
    k, q, p = w1.shape
    ranks = set()
    for lam in range(nb):
        for a in range(nb):
            sv = torch.linalg.svdvals(M[lam::nb, a * p:(a + 1) * p])
            ranks.add(int((sv > 1e-9 * sv[0]).sum()))
    assert ranks == {q // nb}


def test_bf16_inputs_round_each_product_to_bf16():
    """The oracle's products round to the input dtype, like the reference's bf16 bmms: the saved
    intermediate and every result are bf16 and equal the fp32 product rounded once."""
    w1, w2 = factors(64, 64, 4, dtype=torch.float32)
    w1, w2 = w1.bfloat16(), w2.bfloat16()
    x = torch.randn(7, 64, generator=torch.Generator().manual_seed(2)).bfloat16()
    out_blk, out1 = bf.butterfly_fwd(x, w1, w2)
    assert out_blk.dtype == out1.dtype == torch.bfloat16
    k, q, p = w1.shape
    ref1 = torch.bmm(x.float().reshape(7, k, p).transpose(0, 1), w1.float().transpose(-1, -2))
    assert torch.equal(out1, bf.riffle(ref1.bfloat16(), 4))
    dx, dw1, dw2 = bf.butterfly_bwd(x, w1, w2, out1, torch.randn(7, 4, 16).bfloat16())
    assert dx.dtype == dw1.dtype == dw2.dtype == torch.bfloat16
