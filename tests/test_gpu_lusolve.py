"""The FP32 solve of solve(...) (ozaki_jax/solve.py:159, :164): the LU
factorisation with partial pivoting (ozk_lu_factor_f32) and the triangular
solves on a factor (ozk_lu_solve_f32).

The factorisation is checked by what defines it: P A = L U to FP32 rounding
(|P A - L U| <= 8 n eps32 max|A|, a bound that a wrong swap, multiplier or
update exceeds by orders of magnitude), |L| <= 1 (partial pivoting), perm a
permutation, and for n <= 64 the same pivots as LAPACK's sgetrf.

For the solves, the factors come from SciPy's float32 getrf on the CPU, so
the test checks the solves alone: the result is compared with the same triangular solves done in
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


# (4096, 8) and (2100, 8): 8 columns leave 32 workgroups per column for 64
# and 33 row blocks, so one workgroup runs several blocks in order.  (300,
# 300): more columns than compute units, solved in launches of one chunk of
# columns each, one workgroup per column.
CASES = [(1, 1, 0, "dominant"), (5, 1, 0, "randn"), (64, 1, 0, "dominant"),
         (65, 2, 0, "dominant"), (127, 1, 3, "randn"), (300, 3, 0, "dominant"),
         (1000, 1, 0, "randn"), (1000, 2, 1, "dominant"), (2100, 1, 0, "dominant"),
         (4096, 1, 0, "dominant"), (4096, 8, 0, "dominant"), (2100, 8, 1, "randn"),
         (300, 300, 0, "dominant")]


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


def test_lu_solve_subnormal_pivot(ozk):
    """A diagonal entry of U below 2^-128 (its reciprocal overflows FP32):
    that row block is solved unscaled, dividing in the chain, so the zeros
    of its rows stay zeros and the solution stays finite."""
    rng = np.random.RandomState(9)
    n = 200
    lu = np.triu(rng.randn(n, n) * 0.1 + np.diag(2.0 + rng.rand(n))).astype(np.float32)
    lu[10, 11:] = 0.0
    lu[10, 10] = np.float32(1e-39)        # subnormal pivot
    b = rng.randn(n, 1)
    b[10, 0] = float(np.float32(3e-39))
    perm = np.arange(n, dtype=np.int32)
    case("ozk_lu_solve_f32 subnormal pivot")
    X = gpu_solve(lu, perm, b)
    Xr = ref_solve(lu, perm, b)
    assert np.isfinite(X).all() and abs(X[10, 0] - 3.0) < 1e-5
    assert np.linalg.norm(X - Xr) <= 2e-5 * np.linalg.norm(Xr)


def test_solve_eight_columns_n4096(ozk):
    """solve() with an 8-column right-hand side at n = 4096: the native
    solves with several row blocks per workgroup.  The refined error against
    LAPACK's FP64 answer (bounded by the high preset's residual accuracy at
    rho = 18) is within 2x of the oracle's refinement.  (The matrix is so well
    conditioned that refinement gains little over the FP32 solve; the
    condition-1e6 test separates refined from unrefined answers.)"""
    import oracle as O
    rng = np.random.RandomState(12)
    n = 4096
    A = dominant(n, rng)
    B = rng.randn(n, 8)
    case("solve ozaki n=4096 with 8 right-hand sides")
    X = ozk.solve(A, B, residual_mode="ozaki")
    Xr = np.linalg.solve(A, B)
    assert X.shape == (n, 8)

    def err(x):
        return np.linalg.norm(x - Xr) / np.linalg.norm(Xr)

    assert err(X) <= 2.0 * err(O.solve_ozaki(A, B))


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


def test_lu_solve_workspace_reused(ozk):
    """One workspace through calls of different sizes: each call clears the
    published words it polls, so what an earlier call left there (solution
    words of a larger system, tagged as ready) is never read as a result."""
    import torch
    from ozaki_jax_amd import _device as D, _lib
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    rng = np.random.RandomState(21)
    wsb = lib.ozk_lu_solve_workspace_bytes(700, 3)
    ws = D.workspace(wsb, dev)
    flags = torch.zeros(1, dtype=torch.int32, device=dev)
    for n, nc in [(700, 3), (300, 2), (700, 3), (129, 1)]:
        lu, ipiv = factor(dominant(n, rng))
        perm = perm_of(lib, ipiv)
        B = rng.randn(n, nc)
        case(f"ozk_lu_solve_f32 n={n} ncols={nc} on a shared workspace")
        LUt = torch.from_numpy(np.ascontiguousarray(lu)).to(dev)  # SciPy's is column-major
        Bt = torch.from_numpy(B).to(dev)
        Xt = torch.empty_like(Bt)
        pt = torch.from_numpy(perm).to(dev)
        _lib.check(lib.ozk_lu_solve_f32(LUt.data_ptr(), n, pt.data_ptr(), n, Bt.data_ptr(), nc,
                                        Xt.data_ptr(), nc, nc, ws.data_ptr(), wsb,
                                        flags.data_ptr(), D.stream_handle()))
        assert int(flags.item()) == 0
        Xr = ref_solve(lu, perm, B)
        assert np.linalg.norm(Xt.cpu().numpy() - Xr) <= 2e-5 * np.linalg.norm(Xr)


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


def gpu_factor(A32, pad=0):
    import torch
    from ozaki_jax_amd import _device as D, _lib
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    n = A32.shape[0]
    buf = np.zeros((n, n + pad), np.float32)
    buf[:, :n] = A32
    At = torch.from_numpy(buf).to(dev)
    perm = torch.empty(n, dtype=torch.int32, device=dev)
    flags = torch.full((1,), 7, dtype=torch.int32, device=dev)
    wsb = lib.ozk_lu_factor_workspace_bytes(n)
    ws = D.workspace(wsb, dev)
    _lib.check(lib.ozk_lu_factor_f32(At.data_ptr(), n + pad, n, perm.data_ptr(),
                                     ws.data_ptr(), wsb, flags.data_ptr(),
                                     D.stream_handle()))
    return At.cpu().numpy()[:, :n], perm.cpu().numpy(), int(flags.item())


FACTOR_CASES = [(1, 0), (2, 0), (17, 1), (32, 0), (33, 0), (48, 3), (64, 0), (100, 0),
                (257, 2), (1000, 0), (2048, 1), (4096, 0)]


@pytest.mark.parametrize("n,pad", FACTOR_CASES)
def test_lu_factor_pa_equals_lu(ozk, n, pad):
    rng = np.random.RandomState(100 + n)
    A32 = rng.randn(n, n).astype(np.float32)
    case(f"ozk_lu_factor_f32 n={n} lda=n+{pad}")
    F, perm, flags = gpu_factor(A32, pad)
    assert flags == 0
    assert sorted(perm.tolist()) == list(range(n)), "perm"
    L = np.tril(F.astype(np.float64), -1) + np.eye(n)
    U = np.triu(F.astype(np.float64))
    assert np.abs(np.tril(F, -1)).max(initial=0.0) <= 1.0, "|L| <= 1"
    err = np.abs(A32.astype(np.float64)[perm] - L @ U).max()
    assert err <= 8 * n * np.finfo(np.float32).eps * np.abs(A32).max(), err
    if n <= 64:
        _, piv = sla.lu_factor(A32)
        ps = np.arange(n)
        for i, p in enumerate(piv):
            ps[i], ps[p] = ps[p], ps[i]
        assert np.array_equal(ps, perm), "pivots differ from sgetrf"


def test_lu_factor_singular_flag(ozk):
    from ozaki_jax_amd import _lib
    rng = np.random.RandomState(7)
    A32 = rng.randn(40, 40).astype(np.float32)
    case("ozk_lu_factor_f32 nonsingular: no flag")
    assert gpu_factor(A32)[2] == 0
    A32[:, 20] = 0.0
    case("ozk_lu_factor_f32 zero column: singular flag")
    F, perm, flags = gpu_factor(A32)
    assert flags & _lib.OZK_FLAG_SINGULAR
    assert np.isfinite(F).all() and F[20, 20] == 0.0


def test_solve_n4096_native_factor_and_solves(ozk):
    """The C5 solve shape (n = 4096, condition 1e6) end to end through the
    native factorisation and triangular solves."""
    rng = np.random.RandomState(3)
    n = 4096
    Q1, _ = np.linalg.qr(rng.randn(n, n))
    Q2, _ = np.linalg.qr(rng.randn(n, n))
    A = (Q1 * np.logspace(0, 6, n)) @ Q2.T
    b = rng.randn(n)
    case("solve ozaki n=4096 cond 1e6")
    x = ozk.solve(A, b, residual_mode="ozaki")
    xr = np.linalg.solve(A, b)
    assert np.linalg.norm(x - xr) / np.linalg.norm(xr) <= 1e-3


def test_solve_above_native_lu_limit(ozk):
    """n above ozk_lu_factor_max_n(): torch.linalg's getrf, its pivots turned
    into the permutation by ozk_pivots_to_perm, the library's triangular
    solves on that factor.  Above K = 4096 the high preset's residual is
    accurate to about 4e-8 relative (rho = 19; the oracle's residual agrees bit
    for bit), which bounds what the refinement reaches; f64 residuals reach
    FP64 accuracy through the same factor."""
    from ozaki_jax_amd import _lib
    n = int(_lib.load().ozk_lu_factor_max_n()) + 7
    rng = np.random.RandomState(11)
    A = dominant(n, rng)
    b = rng.randn(n)
    xr = np.linalg.solve(A, b)
    case(f"solve ozaki n={n} (library getrf)")
    x = ozk.solve(A, b, residual_mode="ozaki")
    assert np.linalg.norm(x - xr) / np.linalg.norm(xr) <= 1e-5
    case(f"solve f64 residuals n={n} (library getrf)")
    x = ozk.solve(A, b)
    assert np.linalg.norm(x - xr) / np.linalg.norm(xr) <= 1e-12
