"""Bounded waits between workgroups, made to give up from the host.

ozk_set_wait_polls(1) limits every wait of the kernels launched afterwards
to (about) one poll: the gangs of the column and long-row extraction (a
member that gives up sets OZK_FLAG_WAIT_TIMEOUT and waits no more, so every
kernel still exits) and the row-block chains of the LU triangular solves.
On the flag after an extraction, the package repeats the call once with the
gangs switched off for the thread (ozk_set_gangs(0): transposed columns and
streamed rows, no waits between workgroups), so matmul, gram, residual and
lowlevel.extract still return the exact result.  solve() redoes a
triangular solve that gave up: on torch.linalg's path for torch input, and
with one workgroup per column (no waits between workgroups) for NumPy input.
After ozk_set_wait_polls(0) the same calls run on the gangs again, with no
repeat.
"""

import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture
def set_polls(ozk):
    from ozaki_jax_amd import _lib
    lib = _lib.load()
    yield lib.ozk_set_wait_polls
    lib.ozk_set_wait_polls(0)


def retries():
    from ozaki_jax_amd import _lib
    return _lib.gang_retries


def check_cols(pl, X, rho, cols):
    hi, lo = O.split_hi_lo(X[:, cols])
    sh, eh = O.extract_cols_f32(hi, rho, 4)
    sl, el = O.extract_cols_f32(lo, rho, 1)
    ref = np.concatenate([sh, sl]).transpose(0, 2, 1) * 2.0 ** (24 - rho)
    assert np.array_equal(pl.counts().cpu().numpy()[:, cols, :X.shape[0]], ref)
    assert np.array_equal(pl.exponents().cpu().numpy()[:, cols],
                          np.concatenate([eh, el]).astype(np.int32))


def check_rows(pl, X, rho, rows):
    hi, lo = O.split_hi_lo(X[rows])
    sh, eh = O.extract_rows_f32(hi, rho, 4)
    sl, el = O.extract_rows_f32(lo, rho, 1)
    ref = np.concatenate([sh, sl]) * 2.0 ** (24 - rho)
    assert np.array_equal(pl.counts().cpu().numpy()[:, rows, :X.shape[1]], ref)
    assert np.array_equal(pl.exponents().cpu().numpy()[:, rows],
                          np.concatenate([eh, el]).astype(np.int32))


def test_column_extraction_gives_up_then_repeats_without_gangs(ozk, set_polls):
    from ozaki_jax_amd import lowlevel as ll
    rng = np.random.RandomState(3)
    X = rng.randn(8192, 512)  # 32 panels, gangs of 16 workgroups
    rho = O.rho_f32(8192)
    cols = np.r_[0:20, 500:512]
    set_polls(1)
    case("ozk_extract_f32_i8 by columns (8192, 512), one poll per wait")
    n0 = retries()
    check_cols(ll.extract(X, 1, rho, 4, 1, i8=True), X, rho, cols)
    assert retries() == n0 + 1
    case("matmul 64 x 8192 x 512, one poll per wait")
    A = rng.randn(64, 8192)
    C = ozk.matmul(A, X, pipeline="ondevice")
    assert retries() == n0 + 2
    assert np.array_equal(C[:, cols], O.matmul_ondevice_a4(A, X[:, cols]))
    case("gram 8192 x 512, one poll per wait")
    G = ozk.gram(X, mode="ozaki")
    assert retries() == n0 + 3
    set_polls(0)
    case("the same calls with the built-in limit")
    check_cols(ll.extract(X, 1, rho, 4, 1, i8=True), X, rho, cols)
    assert np.array_equal(ozk.matmul(A, X, pipeline="ondevice"), C)
    assert np.array_equal(ozk.gram(X, mode="ozaki"), G)
    assert retries() == n0 + 3


def test_long_column_gangs_give_up_then_repeat_without_gangs(ozk, set_polls):
    """Columns of 40000 rows: gangs of 79 workgroups, whose members combine
    the exchange words in batches; after giving up, the repeat transposes."""
    from ozaki_jax_amd import lowlevel as ll
    rng = np.random.RandomState(6)
    X = rng.randn(40000, 48)
    rho = O.rho_f32(40000)
    cols = np.r_[0:5, 40:48]
    set_polls(1)
    case("ozk_extract_f32_i8 by columns (40000, 48), one poll per wait")
    n0 = retries()
    check_cols(ll.extract(X, 1, rho, 4, 1, i8=True), X, rho, cols)
    assert retries() == n0 + 1
    case("gram 40000 x 48, one poll per wait")
    G = ozk.gram(X, mode="ozaki")
    assert retries() == n0 + 2
    set_polls(0)
    case("the same calls with the built-in limit")
    check_cols(ll.extract(X, 1, rho, 4, 1, i8=True), X, rho, cols)
    assert np.array_equal(ozk.gram(X, mode="ozaki"), G)
    assert retries() == n0 + 2


def test_row_extraction_gives_up_then_repeats_without_gangs(ozk, set_polls):
    from ozaki_jax_amd import lowlevel as ll
    rng = np.random.RandomState(4)
    X = rng.randn(256, 131072)  # gangs of 8 workgroups per row
    rho = O.rho_f32(131072)
    rows = np.r_[0:3, 254:256]
    set_polls(1)
    case("ozk_extract_f32_i8 by rows (256, 131072), one poll per wait")
    n0 = retries()
    check_rows(ll.extract(X, 0, rho, 4, 1, i8=True), X, rho, rows)
    assert retries() == n0 + 1
    case("matmul 64 x 70000 x 8 (row gangs for A and the transposed B), one poll per wait")
    A, B = rng.randn(64, 70000), rng.randn(70000, 8)
    C = ozk.matmul(A, B, pipeline="ondevice")
    assert retries() == n0 + 2
    assert np.array_equal(C[:4], O.matmul_ondevice_a4(A[:4], B))
    case("residual 64 x 70000 (GEMM path), one poll per wait")
    x, b = rng.randn(70000), rng.randn(64)
    r = ozk.residual(A, x, b, mode="ozaki")
    assert retries() == n0 + 3
    set_polls(0)
    case("the same calls with the built-in limit")
    check_rows(ll.extract(X, 0, rho, 4, 1, i8=True), X, rho, rows)
    assert np.array_equal(ozk.matmul(A, B, pipeline="ondevice"), C)
    assert np.array_equal(ozk.residual(A, x, b, mode="ozaki"), r)
    assert retries() == n0 + 3


def test_lu_solve_gives_up_and_solve_falls_back(ozk, set_polls):
    import importlib

    import torch
    from ozaki_jax_amd import _device as D, _lib
    S = importlib.import_module("ozaki_jax_amd.solve")  # the module, not solve()
    n = 2100
    rng = np.random.RandomState(5)
    A = rng.randn(n, n) + n * np.eye(n)
    b = rng.randn(n)
    dev = torch.device("cuda", 0)
    At = torch.from_numpy(A).to(dev)
    LU, perm = S.lu_factor_f32(At, dev)
    rhs = torch.from_numpy(b[:, None].copy()).to(dev)
    set_polls(1)
    case(f"ozk_lu_solve_f32 n={n}, one poll per wait")
    _, flags = S.lu_solve_f32(LU, perm, rhs, dev)
    assert D.read_flags(flags) & _lib.OZK_FLAG_WAIT_TIMEOUT
    # the bounds of the solve tests: FP64 residuals reach FP64 accuracy, the
    # Ozaki residual (high, K = 2100) bounds the refinement near 1e-8
    case(f"solve n={n} with the triangular solves giving up (NumPy and torch input)")
    xr = np.linalg.solve(A, b)
    n0 = retries()
    x = ozk.solve(A, b)
    assert retries() > n0  # the NumPy path repeated its solves
    assert np.linalg.norm(x - xr) / np.linalg.norm(xr) <= 1e-12
    x = ozk.solve(A, b, residual_mode="ozaki")
    assert np.linalg.norm(x - xr) / np.linalg.norm(xr) <= 1e-5
    xt = ozk.solve(At, torch.from_numpy(b).to(dev)).cpu().numpy()
    assert np.linalg.norm(xt - xr) / np.linalg.norm(xr) <= 1e-12
    set_polls(0)
    case(f"ozk_lu_solve_f32 n={n}, built-in limit")
    d, flags = S.lu_solve_f32(LU, perm, rhs, dev)
    assert not D.read_flags(flags) & _lib.OZK_FLAG_WAIT_TIMEOUT
    d32 = torch.linalg.solve_triangular(
        LU, torch.linalg.solve_triangular(LU, rhs.to(torch.float32)[perm.long()], upper=False,
                                          unitriangular=True), upper=True)
    assert np.allclose(d.cpu().numpy(), d32.cpu().numpy(), rtol=1e-4, atol=1e-6)
