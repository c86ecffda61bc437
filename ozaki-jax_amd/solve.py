"""Accurate residual and iterative-refinement solve (mirror of
``ozaki_jax/solve.py``).

residual(mode='ozaki') is b - Ozaki(A, x) with the 2Sum order, computed by the
HIP kernels (solve.py:38-53, :78-82).  solve(residual_mode='ozaki') is FP32 LU
plus max_iterations refinement steps whose residuals come from the same
kernels (solve.py:154-167).  The reference's FP32 jnp.linalg.solve becomes
an FP32 LU with partial pivoting, factored once and reused (the reference
re-solves with the same matrix each iteration, which yields the same
factors): ozk_lu_factor_f32 up to n = ozk_lu_factor_max_n() (torch.linalg's
getrf above), then the library's triangular solves (ozk_lu_solve_f32) on that
factor.  mode='f64' paths are plain FP64 products (rocBLAS DGEMM).  NumPy
operands up to n = ozk_lu_factor_max_n() need no PyTorch (device arrays of
the HIP runtime, rocBLAS through ctypes), as in the reference's NumPy use.
"""

from . import _device as D
from . import _lib
from .extract import rho_f32  # noqa: F401  (rho is derived inside the library)
from .matmul import _resolve_precision


def _validate_solve_inputs(A, b):
    """solve.py:22-35."""
    if A.ndim != 2 or A.shape[0] != A.shape[1]:
        raise ValueError(f"A must be square, got shape {tuple(A.shape)}.")
    N = A.shape[0]
    if b.ndim == 1:
        if b.shape[0] != N:
            raise ValueError(f"b length {b.shape[0]} != A size {N}.")
    elif b.ndim == 2:
        if b.shape[0] != N:
            raise ValueError(f"b rows {b.shape[0]} != A size {N}.")
    else:
        raise ValueError(f"b must be 1D or 2D, got ndim={b.ndim}.")


def _validate_residual_inputs(A, x, b):
    """solve.py:55-75."""
    if A.ndim != 2:
        raise ValueError(f"A must be 2D, got ndim={A.ndim}.")
    N, K = A.shape
    if x.ndim == 1:
        if x.shape[0] != K:
            raise ValueError(f"x length {x.shape[0]} != A columns {K}.")
        if b.ndim != 1 or b.shape[0] != N:
            raise ValueError(
                f"b shape {tuple(b.shape)} incompatible with A @ x shape "
                f"({N},).")
    elif x.ndim == 2:
        if x.shape[0] != K:
            raise ValueError(f"x rows {x.shape[0]} != A columns {K}.")
        if b.ndim != 2 or b.shape[0] != N or b.shape[1] != x.shape[1]:
            raise ValueError(
                f"b shape {tuple(b.shape)} incompatible with A @ x shape "
                f"({N}, {x.shape[1]}).")
    else:
        raise ValueError(f"x must be 1D or 2D, got ndim={x.ndim}.")


def _check_mode(mode, accumulation, name):
    allowed = {"f64", "ozaki"}
    if mode not in allowed:
        raise ValueError(f"{name}={mode!r}; expected one of {sorted(allowed)}.")
    if mode == "ozaki":
        allowed_accum = {"bf16_interleaved", "fused"}
        if accumulation not in allowed_accum:
            raise ValueError(
                f"accumulation={accumulation!r}; expected one of "
                f"{sorted(allowed_accum)}.")


def _asarray(v):
    if D.is_torch(v):
        return v
    import numpy as np
    return np.asarray(v)


def ozaki_residual_device(fam, At, xt, bt, n_hi, n_lo):
    """r = b - Ozaki(A, x) on device arrays of family `fam` (x, b 2-D)."""
    lib = _lib.load()
    N, K = At.shape
    nc = xt.shape[1]
    r = fam.empty((N, nc))
    if N == 0 or nc == 0:
        return r
    if K == 0:
        raise ValueError("zero-size array to reduction operation maximum "
                         "which has no identity")
    flags = fam.flags()  # ozk_residual clears the flag word itself
    fused = lib.ozk_residual_workspace_bytes(N, K, nc, n_hi, n_lo) == 0

    def once():
        wsb = lib.ozk_residual_workspace_bytes(N, K, nc, n_hi, n_lo)
        ws = fam.workspace(wsb)
        _lib.check(lib.ozk_residual(
            At.data_ptr(), D.ld_of(At), xt.data_ptr(), D.ld_of(xt), bt.data_ptr(),
            D.ld_of(bt), r.data_ptr(), D.ld_of(r), N, K, nc, n_hi, n_lo,
            ws.data_ptr(), wsb, flags.data_ptr(), fam.stream()))
        return fam.read_flags(flags)

    if fused and getattr(fam, "early_flags", None) is not None:
        # The fused row kernels (no workspace) have no bounded waits, so the
        # word can hold no OZK_FLAG_WAIT_TIMEOUT, and NaN / Inf are left to
        # propagate as in the reference: a torch result is returned ordered
        # on the current stream, without waiting for the kernel.
        _lib.check(lib.ozk_residual(
            At.data_ptr(), D.ld_of(At), xt.data_ptr(), D.ld_of(xt), bt.data_ptr(),
            D.ld_of(bt), r.data_ptr(), D.ld_of(r), N, K, nc, n_hi, n_lo,
            0, 0, flags.data_ptr(), fam.stream()))
        return r
    _lib.with_gang_retry(once)
    return r


def residual(A, x, b, precision="high", accumulation="bf16_interleaved",
             mode="f64"):
    """solve.py:91-151: b - A @ x; same family and shape as b.  Runs no
    preflight, as the reference: NaN / Inf give NaN entries of r."""
    _check_mode(mode, accumulation, "mode")
    A, x, b = _asarray(A), _asarray(x), _asarray(b)
    want_torch = D.is_torch(A)
    _validate_residual_inputs(A, x, b)
    fam = D.family(want_torch)
    At = fam.f64(A)
    xt = fam.f64(x)
    bt = fam.f64(b)
    vec = xt.dim() == 1
    if vec:
        xt = fam.column(xt)
        bt = fam.column(bt)
    if mode == "f64":
        r = fam.residual_f64(At, xt, bt)
    else:
        n_hi, n_lo = _resolve_precision(precision)
        r = ozaki_residual_device(fam, At, xt, bt, n_hi, n_lo)
    if vec:
        r = fam.flat(r)
    return fam.out(r, want_torch)


def solve(A, b, precision="high", accumulation="bf16_interleaved",
          max_iterations=3, residual_mode="f64"):
    """solve.py:189-257: FP32 LU + iterative refinement."""
    _check_mode(residual_mode, accumulation, "residual_mode")
    A, b = _asarray(A), _asarray(b)
    want_torch = D.is_torch(A)
    _validate_solve_inputs(A, b)
    if not want_torch and not D.is_torch(b) and A.shape[0] <= _lib.load().ozk_lu_factor_max_n():
        return _solve_numpy(A, b, precision, max_iterations, residual_mode)
    dev = D.require_gpu()
    fam = D.family(True)
    torch = D.torch
    At = D.to_device_f64(A, dev)
    bt = D.to_device_f64(b, dev)
    vec = bt.dim() == 1
    if vec:
        bt = bt[:, None].contiguous()
    LU, perm = lu_factor_f32(At, dev)

    def solve_trsm(rhs):  # BLAS-3 triangular solves on the same factor
        y = torch.linalg.solve_triangular(LU, rhs.to(torch.float32)[perm.long()],
                                          upper=False, unitriangular=True)
        return torch.linalg.solve_triangular(LU, y, upper=True).to(torch.float64)

    def solve32(rhs):
        if rhs.shape[1] > LU_SOLVE_MAX_COLS:  # many columns (inv)
            return solve_trsm(rhs)
        d, flags = lu_solve_f32(LU, perm, rhs, dev)
        # A row block that gave up waiting (the GPU shared with other work
        # long enough to stall the chain) leaves d invalid: redo this solve.
        if D.read_flags(flags) & _lib.OZK_FLAG_WAIT_TIMEOUT:
            return solve_trsm(rhs)
        return d

    x = solve32(bt)
    if residual_mode == "ozaki":
        n_hi, n_lo = _resolve_precision(precision)
    for _ in range(max_iterations):
        if residual_mode == "f64":
            r = bt - torch.matmul(At, x)
        else:
            r = ozaki_residual_device(fam, At, x.contiguous(), bt, n_hi, n_lo)
        x = x + solve32(r)
    if vec:
        x = x[:, 0]
    return D.to_family(x, want_torch)


def _solve_numpy(A, b, precision, max_iterations, residual_mode):
    """solve() for NumPy operands of n <= ozk_lu_factor_max_n(), with no
    PyTorch: device arrays of the HIP runtime, the library's FP32 LU and
    triangular solves, rocBLAS for the FP64 residual and the update."""
    import numpy as np
    from . import _hip
    lib = _lib.load()
    fam = D.family(False)
    A = np.ascontiguousarray(A, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    vec = b.ndim == 1
    n = A.shape[0]
    At = fam.f64(A)
    bt = fam.f64(b[:, None] if vec else b)
    nc = bt.shape[1]
    if n == 0 or nc == 0:
        return np.zeros(b.shape)
    # A32 = RN32(A) with 16-byte rows, as the torch path's LU.copy_(At)
    lda = max(-(-n // 4) * 4, 4)
    a32 = np.zeros((n, lda), np.float32)
    a32[:, :n] = A
    LU = _hip.DeviceArray.from_numpy(a32)
    perm = fam.empty((n,), np.int32)
    wsb = lib.ozk_lu_factor_workspace_bytes(n)
    ws = fam.workspace(wsb)
    _lib.check(lib.ozk_lu_factor_f32(LU.data_ptr(), lda, n, perm.data_ptr(), ws.data_ptr(),
                                     wsb, fam.flags().data_ptr(), None))

    def solve32(rhs):
        # A row block that gave up waiting (the GPU shared with other work
        # long enough to stall the chain) leaves d invalid: with_gang_retry
        # solves again with one workgroup per column, which waits for no
        # other workgroup.
        d = fam.empty((n, nc))

        def once():
            flags = fam.flags()  # cleared by the call
            wsb = lib.ozk_lu_solve_workspace_bytes(n, nc)
            ws = fam.workspace(wsb)
            _lib.check(lib.ozk_lu_solve_f32(
                LU.data_ptr(), lda, perm.data_ptr(), n, rhs.data_ptr(), D.ld_of(rhs),
                d.data_ptr(), D.ld_of(d), nc, ws.data_ptr(), wsb, flags.data_ptr(), None))
            return fam.read_flags(flags)

        _lib.with_gang_retry(once)
        return d

    blas = _hip.blas()
    x = solve32(bt)
    if residual_mode == "ozaki":
        n_hi, n_lo = _resolve_precision(precision)
    for _ in range(max_iterations):
        if residual_mode == "f64":
            r = fam.residual_f64(At, x, bt)
        else:
            r = ozaki_residual_device(fam, At, x, bt, n_hi, n_lo)
        x = blas.add(x, solve32(r), fam.empty((n, nc)))
    out = x.numpy()
    return out[:, 0] if vec else out


# ozk_lu_solve_f32 solves each right-hand side as its own chain of row
# blocks, re-reading the factor per column; beyond this many columns the
# solve goes to torch.linalg.solve_triangular, whose triangular solves share
# the factor's reads across columns.
LU_SOLVE_MAX_COLS = 8


def lu_factor_f32(At, dev):
    """FP32 LU with partial pivoting of the FP64 device matrix At (the
    factorisation inside the reference's jnp.linalg.solve(A32, .),
    solve.py:159): (LU, perm) with LU an (n, n) row-major FP32 view (unit L
    below the diagonal, U on and above it) and perm the device int32 row
    permutation (row i of P A is row perm[i] of A)."""
    torch = D.torch
    lib = _lib.load()
    n = At.shape[0]
    if n <= lib.ozk_lu_factor_max_n():
        lda = max(-(-n // 4) * 4, 4)  # 16-byte rows for the kernels' vector loads
        LU = torch.empty((n, lda), dtype=torch.float32, device=dev)[:, :n]
        LU.copy_(At)
        perm = torch.empty(n, dtype=torch.int32, device=dev)
        flags = torch.empty(1, dtype=torch.int32, device=dev)  # cleared by the call
        wsb = lib.ozk_lu_factor_workspace_bytes(n)
        ws = D.workspace(wsb, dev)
        _lib.check(lib.ozk_lu_factor_f32(LU.data_ptr(), lda, n, perm.data_ptr(),
                                         ws.data_ptr(), wsb, flags.data_ptr(),
                                         D.stream_handle()))
        return LU, perm
    LU, piv = torch.linalg.lu_factor(At.to(torch.float32))
    LU = LU.contiguous()
    piv_h = piv.to(device="cpu", dtype=torch.int32).contiguous()
    perm_h = torch.empty(n, dtype=torch.int32)
    _lib.check(lib.ozk_pivots_to_perm(piv_h.data_ptr(), n, perm_h.data_ptr()))
    return LU, perm_h.to(dev)


def lu_solve_f32(LU, perm, rhs, dev):
    """d = A32^-1 rhs through ozk_lu_solve_f32 on a factor from
    lu_factor_f32; rhs is an (n, k) FP64 device tensor, d likewise.  Returns
    (d, flags); flags holds OZK_FLAG_WAIT_TIMEOUT if the solve gave up."""
    torch = D.torch
    lib = _lib.load()
    n, nc = rhs.shape
    d = torch.empty((n, nc), dtype=torch.float64, device=dev)
    flags = torch.empty(1, dtype=torch.int32, device=dev)  # cleared by the call
    wsb = lib.ozk_lu_solve_workspace_bytes(n, nc)
    ws = D.workspace(wsb, dev)
    _lib.check(lib.ozk_lu_solve_f32(
        LU.data_ptr(), D.ld_of(LU), perm.data_ptr(), n, rhs.data_ptr(),
        D.ld_of(rhs), d.data_ptr(), D.ld_of(d), nc, ws.data_ptr(), wsb,
        flags.data_ptr(), D.stream_handle()))
    return d, flags
