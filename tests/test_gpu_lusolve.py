"""Triangular solves on an FP32 LU factor (ozk_lu_solve_f32), the FP32 solve
of solve(...) (ozaki_jax/solve.py:159, :164).

The factors come from SciPy's float32 getrf on the CPU, so the test checks the
solves alone: the result is compared with the same triangular solves done in
float64 on the same FP32 factors.  What is left is the kernel's FP32 rounding,
bounded through the factors' conditioning: well-conditioned factors (a
diagonally dominant matrix with its rows shuffled, so that partial pivoting
still permutes) are held to 2e-5, plain N(0, 1) matrices to 1e-3.  A wrong
index, permutation or block dependency gives errors of order one.
"""

import sys

import numpy as np
import pytest
import scipy.linalg as sla

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def factor(A):
    """float32 getrf (SciPy, 0-based pivots) -> (LU, LAPACK 1-based ipiv)."""
    lu, piv = sla.lu_factor(A.astype(np.float32))
    return lu.astype(np.float32), (piv + 1).astype(np.int32)


def ref_solve(lu, perm, B):
    """x = U^-1 L^-1 (B[perm]) in float64 on the FP32 factors."""
    L = np.tril(lu.astype(np.float64), -1) + np.eye(lu.shape[0])
    U = np.triu(lu.astype(np.float64))
    y = sla.solve_triangular(L, B.astype(np.float32).astype(np.float64)[perm],
                             lower=True, unit_diagonal=True)
    return sla.solve_triangular(U, y, lower=False)


def gpu_solve(lu, perm, B, pad=0, alias=False):
    import torch
    from ozaki_jax_amd import _device as D, _lib
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    n, nc = B.shape
    LUp = np.zeros((n, n + pad), np.float32)
    LUp[:, :n] = lu
    LUt = torch.from_numpy(LUp).to(dev)
    Bt = torch.from_numpy(np.ascontiguousarray(B)).to(dev)
    Xt = Bt if alias else torch.empty_like(Bt)
    pt = torch.from_numpy(perm).to(dev)
    flags = torch.full((1,), 7, dtype=torch.int32, device=dev)
    wsb = lib.ozk_lu_solve_workspace_bytes(n, nc)
    ws = D.workspace(wsb, dev)
    _lib.check(lib.ozk_lu_solve_f32(LUt.data_ptr(), n + pad, pt.data_ptr(), n,
                                    Bt.data_ptr(), nc, Xt.data_ptr(), nc, nc,
                                    ws.data_ptr(), wsb, flags.data_ptr(),
                                    D.stream_handle()))
    assert int(flags.item()) == 0, "flags"
    return Xt.cpu().numpy()


def perm_of(lib, ipiv):
    n = len(ipiv)
    perm = np.empty(n, np.int32)
    assert lib.ozk_pivots_to_perm(ipiv.ctypes.data, n, perm.ctypes.data) == 0
    return perm


def dominant(n, rng):
    """Diagonal 2..3 plus N(0, 0.25 / n) entries (row norm about 0.5):
    condition number about 2 at every n; rows shuffled."""
    A = rng.randn(n, n) * (0.5 / np.sqrt(n)) + np.diag(2.0 + rng.rand(n))
    return A[rng.permutation(n)]


CASES = [(1, 1, 0, "dominant"), (5, 1, 0, "randn"), (64, 1, 0, "dominant"),
         (65, 2, 0, "dominant"), (127, 1, 3, "randn"), (300, 3, 0, "dominant"),
         (1000, 1, 0, "randn"), (1000, 2, 1, "dominant"), (2100, 1, 0, "dominant"),
         (4096, 1, 0, "dominant")]


@pytest.mark.parametrize("n,nc,pad,kind", CASES)
def test_lu_solve_matches_float64_solves(ozk, n, nc, pad, kind):
    from ozaki_jax_amd import _lib
    lib = _lib.load()
    rng = np.random.RandomState(n + 17 * nc)
    A = dominant(n, rng) if kind == "dominant" else rng.randn(n, n)
    lu, ipiv = factor(A)
    perm = perm_of(lib, ipiv)
    B = rng.randn(n, nc)
    case(f"ozk_lu_solve_f32 n={n} ncols={nc} lda=n+{pad} {kind}")
    X = gpu_solve(lu, perm, B, pad=pad)
    Xr = ref_solve(lu, perm, B)
    err = np.linalg.norm(X - Xr) / np.linalg.norm(Xr)
    assert err <= (2e-5 if kind == "dominant" else 1e-3), err


def test_lu_solve_in_place_and_empty(ozk):
    from ozaki_jax_amd import _lib
    lib = _lib.load()
    rng = np.random.RandomState(5)
    n = 200
    lu, ipiv = factor(dominant(n, rng))
    perm = perm_of(lib, ipiv)
    B = rng.randn(n, 2)
    case("ozk_lu_solve_f32 X aliasing B")
    X = gpu_solve(lu, perm, B, alias=True)
    assert np.linalg.norm(X - ref_solve(lu, perm, B)) <= 2e-5 * np.linalg.norm(X)
    case("ozk_lu_solve_f32 with no right-hand side")
    assert gpu_solve(lu, perm, np.zeros((n, 0))).shape == (n, 0)


def test_solve_uses_native_triangular_solves(ozk):
    """solve() at one right-hand side goes through ozk_lu_solve_f32 and
    matches LAPACK's FP64 answer on a matrix of condition 1e6 (the C5 form)."""
    rng = np.random.RandomState(3)
    n = 512
    Q1, _ = np.linalg.qr(rng.randn(n, n))
    Q2, _ = np.linalg.qr(rng.randn(n, n))
    A = (Q1 * np.logspace(0, 6, n)) @ Q2.T
    b = rng.randn(n)
    case("solve ozaki n=512 cond 1e6")
    x = ozk.solve(A, b, residual_mode="ozaki")
    xr = np.linalg.solve(A, b)
    assert np.linalg.norm(x - xr) / np.linalg.norm(xr) <= 1e-4
