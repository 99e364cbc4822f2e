"""HIP butterfly forward/backward (mmuon_butterfly_fwd / _bwd through the C ABI) against the
oracle (oracle/butterfly.py, pinned by tests/test_oracle_butterfly.py).

Inputs are bf16, the oracle multiplies the same bf16 values in fp32 and rounds each product to
bf16 where the reference's bmms round.  Only the summation order differs, so an output element
differs by at most a bf16 rounding step where the fp32 sums straddle one.  Bar: relative Frobenius
error <= 2e-3 per output, five times tighter than the bf16 tolerance of the optimizer path (1e-2);
the measured errors are printed and sit between 2e-5 and 2e-4.  Shapes: the Monarch factors of
the benchmark models (toy nb=2, 257M nb=2, 1.3B nb=4, 6.89B nb=4: square, tall-w2 and wide-w1
layers), token counts that are not multiples of the 256-row tile, split-K weight gradients with a
ragged last split, and the empty and single-token edge cases.
"""
import pytest
import torch

from monarch_muon_amd import butterfly_blk, butterfly_blk_bwd_op, butterfly_blk_op
from oracle import butterfly as bf
from oracle.truth import rel_fro

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
TOL = 2e-3

# (tokens, nblocks, q, p, s): w1 (nb, q, p), w2 (nb, s, q), x (tokens, nb p)
CASES = [
    (1000, 2, 256, 256, 688),     # toy gate/up (in 512 -> out 1376)
    (1000, 2, 256, 688, 256),     # toy down
    (700, 2, 512, 512, 1368),     # 257M up
    (700, 2, 512, 1368, 512),     # 257M down
    (600, 4, 512, 512, 1376),     # 1.3B up
    (512, 4, 1024, 1024, 1024),   # 6.89B q/k/v/o
    (300, 4, 1024, 1024, 2752),   # 6.89B gate/up
    (300, 4, 1024, 2752, 1024),   # 6.89B down
    (5000, 4, 256, 256, 256),     # split-K weight gradients, ragged last split
    (1, 4, 256, 256, 256),
    (300, 1, 256, 512, 384),      # one block: the riffle is the identity
    (200, 8, 256, 256, 264),      # eight blocks: 32-column planes, s not a multiple of 16
    (200, 16, 512, 256, 520),     # sixteen blocks (the most the kernels take): 16-column planes
]


def make(tokens, nb, q, p, s, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(tokens, nb * p, generator=g).bfloat16()
    w1 = (torch.randn(nb, q, p, generator=g) / p ** 0.5).bfloat16()
    w2 = (torch.randn(nb, s, q, generator=g) / q ** 0.5).bfloat16()
    dout = torch.randn(tokens, nb, s, generator=g).bfloat16()
    return x, w1, w2, dout


def gpu(*ts):
    return [t.to(DEV) for t in ts]


def rel(a, b):
    return float(rel_fro(a.detach().cpu().double().reshape(1, 1, -1), b.detach().cpu().double().reshape(1, 1, -1)).max())


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c)))
def test_forward_and_backward_match_oracle(case):
    print("butterfly case", case, flush=True)
    x, w1, w2, dout = make(*case)
    ref_out, ref_out1 = bf.butterfly_fwd(x, w1, w2)
    ref_dx, ref_dw1, ref_dw2 = bf.butterfly_bwd(x, w1, w2, ref_out1, dout)
    xg, w1g, w2g, dg = gpu(x, w1, w2, dout)
    out, out1 = butterfly_blk_op(xg, w1g, w2g)
    # the backward from the oracle's intermediate, so each op is checked on its own inputs
    dx, dw1, dw2 = butterfly_blk_bwd_op(xg, w1g, w2g, ref_out1.to(DEV), dg)
    torch.cuda.synchronize()
    errs = {"out1": rel(out1, ref_out1), "out": rel(out, ref_out), "dx": rel(dx, ref_dx),
            "dw1": rel(dw1, ref_dw1), "dw2": rel(dw2, ref_dw2)}
    print(case, {k: f"{v:.2e}" for k, v in errs.items()})
    assert out.shape == ref_out.shape and out1.shape == ref_out1.shape
    for k, v in errs.items():
        assert v <= TOL, (k, v)


def test_zero_tokens():
    x, w1, w2, dout = make(0, 4, 256, 256, 256)
    xg, w1g, w2g, dg = gpu(x, w1, w2, dout)
    out, out1 = butterfly_blk_op(xg, w1g, w2g)
    dx, dw1, dw2 = butterfly_blk_bwd_op(xg, w1g, w2g, out1, dg)
    torch.cuda.synchronize()
    assert out.shape == (0, 4, 256) and out1.shape == (4, 0, 256) and dx.shape == (0, 1024)
    assert not dw1.abs().any() and not dw2.abs().any()


def test_results_are_deterministic():
    x, w1, w2, dout = gpu(*make(2600, 4, 256, 512, 256, seed=7))
    a = butterfly_blk_op(x, w1, w2)
    b = butterfly_blk_op(x, w1, w2)
    ga = butterfly_blk_bwd_op(x, w1, w2, a[1], dout)
    gb = butterfly_blk_bwd_op(x, w1, w2, b[1], dout)
    torch.cuda.synchronize()
    for u, v in zip(a + ga, b + gb):
        assert torch.equal(u, v)


def test_autograd_through_butterfly_blk_under_autocast():
    """fp32 parameters under bf16 autocast, as the reference trains: butterfly_blk casts, the
    custom op's backward runs, the gradients land in fp32 on the parameters."""
    tokens, nb, q, p, s = 384, 4, 512, 512, 1376
    x, w1, w2, _ = make(tokens, nb, q, p, s, seed=11)
    dy = torch.randn(tokens, s * nb, generator=torch.Generator().manual_seed(12)).bfloat16()
    xg = x.float().to(DEV).requires_grad_()
    w1g = w1.float().to(DEV).requires_grad_()
    w2g = w2.float().to(DEV).requires_grad_()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = butterfly_blk(xg.reshape(3, 128, nb * p), w1g, w2g)
    assert y.shape == (3, 128, s * nb) and y.dtype == torch.bfloat16
    y.backward(dy.reshape(3, 128, -1).to(DEV))
    torch.cuda.synchronize()
    ref_y = bf.butterfly_blk(x, w1, w2)
    _, ref_out1 = bf.butterfly_fwd(x, w1, w2)
    ref_dx, ref_dw1, ref_dw2 = bf.butterfly_bwd(x, w1, w2, ref_out1, bf.blocked_grad(dy, nb))
    assert w1g.grad.dtype == torch.float32
    assert rel(y.reshape(tokens, -1), ref_y) <= TOL
    assert rel(xg.grad, ref_dx) <= TOL
    assert rel(w1g.grad, ref_dw1) <= TOL
    assert rel(w2g.grad, ref_dw2) <= TOL


def test_full_size_layer_against_fp32_products():
    """6.89B gate/up layer at the benchmark's 4096 tokens: the oracle's products run on the GPU in
    fp32 (same rounding points) as the checker at this size."""
    x, w1, w2, dout = gpu(*make(4096, 4, 1024, 1024, 2752, seed=5))
    out, out1 = butterfly_blk_op(x, w1, w2)
    dx, dw1, dw2 = butterfly_blk_bwd_op(x, w1, w2, out1, dout)
    ref_out, ref_out1 = bf.butterfly_fwd(x, w1, w2)
    ref = bf.butterfly_bwd(x, w1, w2, ref_out1, dout)
    torch.cuda.synchronize()
    assert rel(out1, ref_out1) <= TOL and rel(out, ref_out) <= TOL
    for u, v in zip((dx, dw1, dw2), ref):
        assert rel(u, v) <= TOL


def test_rejects_what_the_kernels_do_not_cover():
    x, w1, w2, _ = gpu(*make(16, 4, 256, 256, 256))
    with pytest.raises(TypeError, match="bfloat16"):
        butterfly_blk_op(x.float(), w1.float(), w2.float())
    xb, w1b, w2b, _ = gpu(*make(16, 4, 64, 64, 64))   # q / nblocks = 16, not a multiple of 32
    with pytest.raises(RuntimeError, match="multiple of 32"):
        butterfly_blk_op(xb, w1b, w2b)
