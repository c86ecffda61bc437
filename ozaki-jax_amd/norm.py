"""FP64-accurate norms (mirror of ``ozaki_jax/norm.py``).

Most orders are plain FP64 reductions: on the GPU through torch for torch
input, with NumPy for NumPy input (no PyTorch needed).  The spectral norm
(ord=2) is sqrt(lambda_max(A^T A)) from the accurate Gram matrix: with
mode='ozaki' that Gram matrix comes from the HIP Ozaki kernels (for either
family), and the eigenvalues of the small Gram matrix from torch.linalg or
NumPy's LAPACK respectively."""

import numpy as np

from . import _device as D
from .gram import gram

_INF = float("inf")


class _NumpyOps:
    """The few torch calls of the norms, over NumPy arrays."""
    sqrt, sum, abs, max, min = np.sqrt, np.sum, np.abs, np.max, np.min
    float64 = np.float64
    linalg = np.linalg

    @staticmethod
    def clamp(v, min):
        return np.maximum(v, min)


def _vector_norm(x, ord, t):
    """norm.py:22-35."""
    if ord is None or ord == 2:
        return t.sqrt(t.sum(t.abs(x) ** 2))
    if ord == 1:
        return t.sum(t.abs(x))
    if ord == _INF:
        return t.max(t.abs(x))
    if ord == -_INF:
        return t.min(t.abs(x))
    if ord == 0:
        n = t.sum(x != 0)
        return n.to(t.float64) if t is not _NumpyOps else np.float64(n)
    if isinstance(ord, str):
        raise ValueError(f"Invalid norm order {ord!r} for a vector.")
    return t.sum(t.abs(x) ** ord) ** (1.0 / ord)


def _matrix_norm(A, ord, precision, accumulation, mode, t):
    """norm.py:38-58."""
    if ord is None or ord == "fro":
        return t.sqrt(t.sum(t.abs(A) ** 2))
    if ord == 1:
        return t.max(t.sum(t.abs(A), 0))
    if ord == -1:
        return t.min(t.sum(t.abs(A), 0))
    if ord == _INF:
        return t.max(t.sum(t.abs(A), 1))
    if ord == -_INF:
        return t.min(t.sum(t.abs(A), 1))
    if ord == 2:
        # Largest singular value = sqrt(lambda_max(A^T A)), negative rounding
        # residue clipped (norm.py:50-54).
        G = gram(A, precision=precision, accumulation=accumulation, mode=mode)
        lam = t.linalg.eigvalsh(G)[-1]
        return t.sqrt(t.clamp(lam, min=0.0))
    raise ValueError(
        f"Invalid / unsupported norm order {ord!r} for a matrix. "
        "Supported: 'fro', 1, -1, 2, inf, -inf.")


def norm(x, ord=None, precision="high", accumulation="bf16_interleaved",
         mode="f64"):
    """norm.py:61-102.  A float64 scalar for NumPy input, a 0-d float64
    tensor for torch input."""
    want_torch = D.is_torch(x)
    if not want_torch:
        x = np.asarray(x, dtype=np.float64)
        if x.ndim not in (1, 2):
            raise ValueError(f"x must be 1D or 2D, got ndim={x.ndim}.")
        if x.ndim == 1:
            return np.float64(_vector_norm(x, ord, _NumpyOps))
        return np.float64(_matrix_norm(x, ord, precision, accumulation, mode, _NumpyOps))
    dev = D.require_gpu()
    if x.ndim not in (1, 2):
        raise ValueError(f"x must be 1D or 2D, got ndim={x.ndim}.")
    xt = D.to_device_f64(x, dev)
    if xt.dim() == 1:
        return _vector_norm(xt, ord, D.torch)
    return _matrix_norm(xt, ord, precision, accumulation, mode, D.torch)


__all__ = ["norm"]
