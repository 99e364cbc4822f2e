"""fp64 closed forms that pin the Newton-Schulz restatement -- test infrastructure.

* ``quintic_scalar``: the scalar map x -> a x + b x^3 + c x^5 iterated five
  times.  For X = U diag(s) V^T, the Newton-Schulz output is
  U diag(phi(s / ||s||_2)) V^T (the iteration acts on singular values only),
  which is the known answer used by the tests.
* ``ns_fp64``: the same iteration in float64 (the "truth" against which the
  bf16 error of any implementation is measured).
"""
from __future__ import annotations

import numpy as np
import torch

from .step import NS_COEFFS, NS_EPS, NS_STEPS


def quintic_scalar(x: np.ndarray, steps: int = NS_STEPS) -> np.ndarray:
    a, b, c = NS_COEFFS
    x = np.asarray(x, dtype=np.float64)
    for _ in range(steps):
        x = a * x + b * x ** 3 + c * x ** 5
    return x


def ns_fp64(stack: torch.Tensor) -> torch.Tensor:
    """Newton-Schulz of a ``(N, r, c)`` stack in float64 (three-product form)."""
    x = stack.to(torch.float64)
    x = x / (torch.linalg.matrix_norm(x, ord="fro", keepdim=True) + NS_EPS)
    tall = x.shape[-2] > x.shape[-1]
    if tall:
        x = x.transpose(-2, -1)
    a, b, c = NS_COEFFS
    for _ in range(NS_STEPS):
        A = x @ x.transpose(-2, -1)
        B = b * A + c * (A @ A)
        x = a * x + B @ x
    if tall:
        x = x.transpose(-2, -1)
    return x


def known_answer(u: torch.Tensor, s: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """U diag(phi(s/||s||)) V^T for orthonormal-column U (r x k), V (c x k)."""
    sn = s.to(torch.float64) / (torch.linalg.vector_norm(s.to(torch.float64)) + NS_EPS)
    phi = torch.from_numpy(quintic_scalar(sn.numpy()))
    return (u.to(torch.float64) * phi) @ v.to(torch.float64).transpose(-2, -1)


def rel_fro(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Per-block relative Frobenius error ||a-b|| / ||b|| over the last two dims."""
    a = a.to(torch.float64)
    b = b.to(torch.float64)
    num = torch.linalg.matrix_norm(a - b, ord="fro")
    den = torch.linalg.matrix_norm(b, ord="fro").clamp_min(1e-300)
    return num / den
