"""FP64-accurate inverse (mirror of ``ozaki_jax/inv.py``): A X = I by the
iterative-refinement solve, whose residuals run in the HIP kernels when
residual_mode='ozaki'."""

import numpy as np

from . import _device as D
from .solve import solve


def inv(A, precision="high", accumulation="bf16_interleaved",
        max_iterations=3, residual_mode="f64"):
    """inv.py:11-45."""
    if A.ndim != 2 or A.shape[0] != A.shape[1]:
        raise ValueError(f"A must be square, got shape {tuple(A.shape)}.")
    N = A.shape[0]
    if D.is_torch(A):
        eye = D.torch.eye(N, dtype=D.torch.float64, device=A.device)
    else:
        eye = np.eye(N)
    return solve(A, eye, precision=precision, accumulation=accumulation,
                 max_iterations=max_iterations, residual_mode=residual_mode)


__all__ = ["inv"]
