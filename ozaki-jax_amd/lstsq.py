"""FP64-accurate least squares (mirror of ``ozaki_jax/lstsq.py``).

min ||A x - b||_2 for full-rank A with rows >= cols, by refinement of the
augmented (Bjorck) system over one FP32 QR factorisation (lstsq.py:1-20).
The FP32 QR and triangular solves are library dependencies (torch.linalg on
the GPU, as the reference uses jnp.linalg); with residual_mode='ozaki' the
two residual products A x and A^T r run in the HIP Ozaki kernels, both with
rho sized for the larger dimension (lstsq.py:165-167).
"""

import numpy as np

from . import _device as D
from . import _lib
from . import lowlevel as ll
from .extract import rho_f32
from .matmul import _resolve_precision

_PRESETS = ((4, 1), (3, 1), (5, 4))


def _validate_lstsq_inputs(A, b):
    """lstsq.py:30-47."""
    if A.ndim != 2:
        raise ValueError(f"A must be 2D, got ndim={A.ndim}.")
    M, N = A.shape
    if M < N:
        raise ValueError(
            f"lstsq requires rows >= cols (got {M}x{N}); underdetermined "
            "systems are not supported.")
    if b.ndim == 1:
        if b.shape[0] != M:
            raise ValueError(f"b length {b.shape[0]} != A rows {M}.")
    elif b.ndim == 2:
        if b.shape[0] != M:
            raise ValueError(f"b rows {b.shape[0]} != A rows {M}.")
    else:
        raise ValueError(f"b must be 1D or 2D, got ndim={b.ndim}.")


class _OzakiOperator:
    """A x and A^T r by the Ozaki kernels (order 2Sum, lstsq.py:95-112):
    A's row planes and column planes are extracted once with one rho; each
    right-hand side is extracted by columns per product."""

    def __init__(self, At, rho, n_hi, n_lo):
        self.rho, self.n_hi, self.n_lo = rho, n_hi, n_lo
        self.i8 = rho >= 19 and (n_hi, n_lo) in _PRESETS
        self.rows = ll.extract(At, 0, rho, n_hi, n_lo, i8=self.i8)   # lines: rows of A
        self.cols = ll.extract(At, 1, rho, n_hi, n_lo, i8=self.i8)   # lines: rows of A^T

    def _prod(self, pa, X):
        pb = ll.extract(X, 1, self.rho, self.n_hi, self.n_lo, i8=self.i8)
        return ll.gemm(pa, pb, _lib.PIPE_ONDEVICE, self.n_hi, self.n_lo, _lib.ORDER_2SUM)

    def matvec(self, X):
        return self._prod(self.rows, X)

    def rmatvec(self, R):
        return self._prod(self.cols, R)


def lstsq(A, b, precision="high", accumulation="bf16_interleaved",
          max_iterations=3, residual_mode="f64"):
    """lstsq.py:115-172.  x (N,) or (N, K) in A's family."""
    allowed_residual = {"f64", "ozaki"}
    if residual_mode not in allowed_residual:
        raise ValueError(
            f"residual_mode={residual_mode!r}; expected one of "
            f"{sorted(allowed_residual)}.")
    if residual_mode == "ozaki":
        allowed_accum = {"bf16_interleaved", "fused"}
        if accumulation not in allowed_accum:
            raise ValueError(
                f"accumulation={accumulation!r}; expected one of "
                f"{sorted(allowed_accum)}.")
    want_torch = D.is_torch(A)
    if not D.is_torch(A):
        A = np.asarray(A)
    if not D.is_torch(b):
        b = np.asarray(b)
    _validate_lstsq_inputs(A, b)
    dev = D.require_gpu()
    torch = D.torch
    f32, f64 = torch.float32, torch.float64
    At = D.to_device_f64(A, dev)
    bt = D.to_device_f64(b, dev)
    vec = bt.dim() == 1
    if vec:
        bt = bt[:, None]
    M, N = At.shape

    Q, R = torch.linalg.qr(At.to(f32), mode="reduced")

    def ls_solve(rhs):  # lstsq.py:50-53
        z = Q.T @ rhs.to(f32)
        return torch.linalg.solve_triangular(R, z, upper=True).to(f64)

    def correction(f, g):  # lstsq.py:56-67
        Qtf = Q.T @ f.to(f32)
        Rtg = torch.linalg.solve_triangular(R.T, g.to(f32), upper=False)
        dx = torch.linalg.solve_triangular(R, Qtf - Rtg, upper=True)
        dr = f.to(f32) - Q @ (R @ dx)
        return dr.to(f64), dx.to(f64)

    if residual_mode == "f64":  # lstsq.py:70-84
        def matvec(X):
            return At @ X

        def rmatvec(Rr):
            return At.T @ Rr
    else:  # lstsq.py:87-112
        n_hi, n_lo = _resolve_precision(precision)
        op = _OzakiOperator(At, rho_f32(max(M, N)), n_hi, n_lo)
        matvec, rmatvec = op.matvec, op.rmatvec

    x = ls_solve(bt)
    r = bt - matvec(x)
    for _ in range(max_iterations):
        f = bt - r - matvec(x)
        g = -rmatvec(r)
        dr, dx = correction(f, g)
        x = x + dx
        r = r + dr
    if vec:
        x = x[:, 0]
    return D.to_family(x, want_torch)


__all__ = ["lstsq"]
