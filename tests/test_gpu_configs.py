"""Parity at the benchmark configurations, through the public API.

Each configuration runs at its full size on the GPU; the oracle (NumPy, in
the same accumulation order) checks sampled rows or columns, which are
independent of the others (per-line exponents), plus a full product at a
reduced width.  Bar: bit-exact (np.array_equal), and for the products of the
sampled lines the exactness certificate (every partial sum below 2^24 grid
units), so the FP32 products the reference forms are order-independent.

  long-K   matmul high 1024 x 65536 x 1024, (U - 0.5) exp(2 N) entries (rho 20)
  gram     gram(A, mode='ozaki', precision='high') on 32768 x 2048 N(0,1)
           (rho from A.shape[0] = 32768: 20; K-split tail of 16 tiles)
  wide     matmul medium / max at K = 8192, a_ij = (U - 0.5) exp(phi N)
           with phi_A, phi_B in {0.5, 4}: 48 x 8192 x 40 in full, and
           8192^3 on 3 rows for each of the four (phi_A, phi_B) pairs
  C2       matmul high 4096^3 N(0,1) (rho 18, BF16 planes)
  metric   matmul high 8192^3 N(0,1) (rho 19, INT8 planes)
  solve    solve(A, b, residual_mode='ozaki'), n = 4096,
           A = Q1 diag(logspace(0, 6, n)) Q2^T
"""

import sys
import warnings

import numpy as np
import pytest

import oracle as O
from oracle import pipeline as OP

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def wide(rng, shape, phi):
    return (rng.rand(*shape) - 0.5) * np.exp(phi * rng.randn(*shape))


def oracle_a4(A_rows, B, rho, nh, nl):
    """Order-A4 result of the oracle on rows of A (one extraction) and
    whether its products carry the exactness certificate."""
    a, ae, b, be = OP.ondevice_slices(A_rows, B, rho, nh, nl)
    sched = OP.ondevice_schedule(nh, nl)
    unit = 2.0 ** (rho - 24)
    cert = OP.products_exact_certificate(a, b, sched, unit, unit)
    C = OP.combine_f64(*OP.accumulate_a4(OP.slice_products(a, b, sched), sched, ae, be))
    return C, cert


def torch_inputs(A, B):
    import torch
    return (torch.from_numpy(A).to("cuda"), torch.from_numpy(B).to("cuda"))


def test_long_k_1024x65536x1024(ozk):
    rng = np.random.RandomState(0)
    N, K, M = 1024, 65536, 1024
    A, B = wide(rng, (N, K), 2.0), wide(rng, (K, M), 2.0)
    rho = O.rho_f32(K)
    assert rho == 20
    case(f"long-K matmul high ({N},{K},{M}) on device")
    At, Bt = torch_inputs(A, B)
    C = ozk.matmul(At, Bt, pipeline="ondevice", precision="high").cpu().numpy()
    del At, Bt
    rows = np.r_[0:4, 301, 517, 640:644, 700, 811, 1000, N - 3:N]
    assert len(rows) >= 16
    case("long-K oracle on 17 rows (full B extraction on the CPU)")
    ref, cert = oracle_a4(A[rows], B, rho, 4, 1)
    assert cert
    assert np.array_equal(C[rows], ref)
    assert np.all(np.abs(C[rows] - ref) <= 2.0 ** -51 * (np.abs(A[rows]) @ np.abs(B)))


def test_long_k_full_64x65536x48(ozk):
    rng = np.random.RandomState(1)
    A, B = wide(rng, (64, 65536), 2.0), wide(rng, (65536, 48), 2.0)
    case("long-K matmul high (64,65536,48), full product")
    for acc, f in [("fused", O.matmul_ondevice_a4), ("host", O.matmul_ondevice_a3)]:
        C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision="high")
        assert np.array_equal(C, f(A, B)), acc


def test_gram_32768x2048(ozk):
    """Rows and columns of G are independent of each other: G[i, :] comes
    from line i of A's column extraction against all of them, and the
    symmetrised G[i, :] is (G[i, :] + G[:, i]) / 2."""
    import torch
    rng = np.random.RandomState(0)
    A = rng.randn(32768, 2048)
    rho = O.rho_f32(A.shape[0])
    assert rho == 20
    case("gram ozaki high (32768, 2048) on device")
    G = ozk.gram(torch.from_numpy(A).to("cuda"), mode="ozaki").cpu().numpy()
    sel = np.r_[0:3, 64, 777, 1024, 1500, 1983:1988, 2000, 2045:2048]
    assert len(sel) >= 16
    case("gram oracle on 17 rows and columns")
    At = np.ascontiguousarray(A.T)
    g_rows, cert = oracle_a4(At[sel], A, rho, 4, 1)
    g_cols = OP._ozaki_a4_unchecked(At, np.ascontiguousarray(A[:, sel]), rho, 4, 1)
    ref = (g_rows + g_cols.T) * 0.5
    assert cert
    assert np.array_equal(G[sel], ref)
    assert np.array_equal(G, G.T)


def test_gram_full_32768x128(ozk):
    A = np.random.RandomState(2).randn(32768, 128)
    case("gram ozaki high (32768, 128), full")
    G = ozk.gram(A, mode="ozaki")
    assert np.array_equal(G, O.gram_ozaki(A, "high"))


@pytest.mark.parametrize("phi_a,phi_b", [(0.5, 0.5), (0.5, 4.0), (4.0, 0.5), (4.0, 4.0)])
@pytest.mark.parametrize("precision", ["medium", "max"])
def test_wide_range_k8192(ozk, precision, phi_a, phi_b):
    rng = np.random.RandomState(int(10 * phi_a + phi_b))
    A, B = wide(rng, (48, 8192), phi_a), wide(rng, (8192, 40), phi_b)
    nh, nl = OP.resolve_precision(precision)
    for acc, f in [("fused", O.matmul_ondevice_a4), ("host", O.matmul_ondevice_a3)]:
        case(f"matmul {precision} {acc} phi=({phi_a},{phi_b}) (48,8192,40)")
        C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=precision)
        with warnings.catch_warnings(), np.errstate(all="ignore"):
            warnings.simplefilter("ignore")
            ref = f(A, B, "raise", nh, nl)
        assert np.array_equal(C, ref, equal_nan=True)


# 8192^3 wide-range operands, each drawn on its own generator as the
# configuration states, and the oracle's column extraction of each B with
# the max preset's slices (5 hi, 4 lo), whose leading slices are those of
# the medium preset: the extraction is sequential.
_WIDE = {}


def _wide_operand(phi, which):
    key = (phi, which)
    if key not in _WIDE:
        n = 8192
        rs = np.random.RandomState({"A": 40, "B": 41}[which] + int(10 * phi))
        _WIDE[key] = (rs.rand(n, n) - 0.5) * np.exp(phi * rs.randn(n, n))
    return _WIDE[key]


def _wide_b_slices(phi):
    key = (phi, "Bsl")
    if key not in _WIDE:
        B = _wide_operand(phi, "B")
        rho = O.rho_f32(B.shape[0])
        hi, lo = OP.split_hi_lo(B)
        bh, bhe = O.extract_cols_f32(hi, rho, 5)
        bl, ble = O.extract_cols_f32(lo, rho, 4)
        _WIDE[key] = (bh, bhe, bl, ble)
    return _WIDE[key]


def _oracle_rows_b(A_rows, bsl, rho, nh, nl):
    """Order A4 on rows of A against B's precomputed slices."""
    bh, bhe, bl, ble = bsl
    hi, lo = OP.split_hi_lo(A_rows)
    ah, ahe = O.extract_rows_f32(hi, rho, nh)
    al, ale = O.extract_rows_f32(lo, rho, nl)
    a, ae = np.concatenate([ah, al]), np.concatenate([ahe, ale])
    b, be = np.concatenate([bh[:nh], bl[:nl]]), np.concatenate([bhe[:nh], ble[:nl]])
    sched = OP.ondevice_schedule(nh, nl)
    with warnings.catch_warnings(), np.errstate(all="ignore"):
        warnings.simplefilter("ignore")
        P = OP.slice_products(a, b, sched)
        return OP.combine_f64(*OP.accumulate_a4(P, sched, ae, be))


@pytest.mark.parametrize("phi_a,phi_b", [(0.5, 0.5), (0.5, 4.0), (4.0, 0.5), (4.0, 4.0)])
@pytest.mark.parametrize("precision", ["medium", "max"])
def test_wide_range_8192_cubed(ozk, precision, phi_a, phi_b):
    n = 8192
    A, B = _wide_operand(phi_a, "A"), _wide_operand(phi_b, "B")
    nh, nl = OP.resolve_precision(precision)
    case(f"matmul {precision} fused 8192^3 phi=({phi_a}, {phi_b}) on device")
    At, Bt = torch_inputs(A, B)
    C = ozk.matmul(At, Bt, pipeline="ondevice", precision=precision).cpu().numpy()
    del At, Bt
    rows = np.r_[0, 4097, n - 1]
    case(f"matmul {precision} oracle on 3 rows, phi=({phi_a}, {phi_b})")
    ref = _oracle_rows_b(A[rows], _wide_b_slices(phi_b), O.rho_f32(n), nh, nl)
    assert np.array_equal(C[rows], ref, equal_nan=True)
    if (phi_a, phi_b) == (4.0, 0.5) and precision == "max":
        # the whole pipeline's oracle on one row pins the helper above
        assert np.array_equal(C[rows[:1]], O.matmul_ondevice_a4(A[rows[:1]], B, "raise", nh, nl),
                              equal_nan=True)


@pytest.mark.parametrize("n,kind", [(4096, "C2 BF16 planes"), (8192, "metric INT8 planes")])
def test_high_square(ozk, n, kind):
    rng = np.random.RandomState(0)
    A, B = rng.randn(n, n), rng.randn(n, n)
    case(f"matmul high fused {n}^3 ({kind}) on device")
    At, Bt = torch_inputs(A, B)
    C = ozk.matmul(At, Bt, pipeline="ondevice", precision="high").cpu().numpy()
    del At, Bt
    rows = np.r_[0, 1, n // 3, n // 2, n // 2 + 1, 2 * n // 3, n - 2, n - 1]
    case(f"matmul high oracle on 8 rows of {n}^3")
    ref, cert = oracle_a4(A[rows], B, O.rho_f32(n), 4, 1)
    assert cert
    assert np.array_equal(C[rows], ref)


def test_solve_n4096_within_twice_the_oracle(ozk):
    """The refined solution's error against LAPACK's FP64 answer is within
    2x of the oracle's (same refinement, NumPy's FP32 LAPACK solve, the
    oracle's Ozaki residuals).  At this condition number the refinement
    reaches its floor (the Ozaki residual's accuracy times the condition)
    after one step, 27x below the unrefined FP32 solve, so a skipped or
    diverging refinement fails."""
    rng = np.random.RandomState(3)
    n = 4096
    Q1, _ = np.linalg.qr(rng.randn(n, n))
    Q2, _ = np.linalg.qr(rng.randn(n, n))
    A = (Q1 * np.logspace(0, 6, n)) @ Q2.T
    b = rng.randn(n)
    xr = np.linalg.solve(A, b)

    def err(x):
        return np.linalg.norm(x - xr) / np.linalg.norm(xr)

    case("solve ozaki n=4096 cond 1e6")
    e_gpu = err(ozk.solve(A, b, residual_mode="ozaki"))
    case("oracle solve_ozaki n=4096")
    e_ref = err(O.solve_ozaki(A, b))
    e_zero = err(O.solve_ozaki(A, b, max_iterations=0))
    print(f"[solve] gpu {e_gpu:.3e}  oracle {e_ref:.3e}  unrefined {e_zero:.3e}", flush=True)
    assert e_gpu <= 2.0 * e_ref
    assert e_ref < e_zero / 10.0  # the bound excludes an unrefined answer
