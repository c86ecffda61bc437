"""Non-finite slices on INT8 planes, against the oracle.

The reference's FP32 extraction gives a line NaN / +-inf slices when
sigma = 0.75 * 2^(rho + c) or 2^-c overflows FP32 (rows scaled by about
2^110, or lo parts below 2^-127), or when the line holds NaN / Inf
(extract.py:130-148); its products, and with them its output row or column,
are then NaN.  At K > 4096 the library runs on INT8 planes, which store such
slices as zeros with the exponent OZK_EXP_NONFINITE and fold their products
as NaN.  Outputs are compared with np.array_equal(equal_nan=True).
"""

import sys
import warnings

import numpy as np
import pytest

import oracle as O
from oracle import pipeline as OP

pytestmark = pytest.mark.gpu

EXP_NONFINITE = -2 ** 31


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ll(ozk):
    from ozaki_jax_amd import lowlevel
    return lowlevel


def quiet(f, *a, **k):
    with warnings.catch_warnings(), np.errstate(all="ignore"):
        warnings.simplefilter("ignore")
        return f(*a, **k)


def edge_operands(N, K, M, seed):
    """A with rows scaled by 2^-110, 2^-103 (lo slices overflow 2^-c only for
    precision='max'), 2^110 (sigma overflows) and 2^-140 (hi part below
    2^-127); B with columns scaled by 2^-112, 2^108 and 2^-100."""
    rng = np.random.RandomState(seed)
    A, B = rng.randn(N, K), rng.randn(K, M)
    A[1] *= 2.0 ** -110
    A[3] *= 2.0 ** -103
    A[5] *= 2.0 ** 110
    A[N - 2] *= 2.0 ** -140
    B[:, 2] *= 2.0 ** -112
    B[:, 4] *= 2.0 ** 108
    B[:, M - 1] *= 2.0 ** -100
    return A, B


# ---------------------------------------------------------------- extraction

@pytest.mark.parametrize("length", [5000, 8192, 40000, 70000, 150000, 300000])
def test_extract_i8_nonfinite_lines(ll, length):
    """Slices of a line up to its first non-finite one (per part) equal the
    oracle's; from there on they are zeros with exponent OZK_EXP_NONFINITE.
    Covers the register kernel (5000, 8192), lines held by 3, 5 and 10
    workgroups (40000, 70000, 150000) and the streaming kernel (300000)."""
    rng = np.random.RandomState(length)
    X = rng.randn(10, length)
    X[1] *= 2.0 ** -110
    X[2] *= 2.0 ** 110
    X[3] *= 2.0 ** -140
    X[4, 7] = np.nan
    X[5, length - 1] = np.inf
    X[6, 3] = 3.0e300            # finite, but its FP32 hi part is inf
    X[7] *= 2.0 ** -103
    X[8] = 0.0
    rho = O.rho_f32(length)
    n0, n1 = 5, 4
    hi, lo = O.split_hi_lo(X)
    sh, eh = quiet(O.extract_rows_f32, hi, rho, n0)
    sl, el = quiet(O.extract_rows_f32, lo, rho, n1)
    for by_cols in (0, 1):
        case(f"ozk_extract_f32_i8 non-finite lines len={length} by_cols={by_cols}")
        pl = ll.extract(X.T.copy() if by_cols else X, by_cols, rho, n0, n1, i8=True)
        q = pl.counts().cpu().numpy()[:, :10, :length].astype(np.float64)
        e = pl.exponents().cpu().numpy()
        for part, (s_ref, e_ref, p0, n) in enumerate([(sh, eh, 0, n0), (sl, el, n0, n1)]):
            for r in range(10):
                bad = [s for s in range(n) if not np.isfinite(s_ref[s, r]).all()]
                first = bad[0] if bad else n
                for s in range(n):
                    if s < first:
                        assert e[p0 + s, r] == e_ref[s, r], (part, r, s)
                        assert np.array_equal(q[p0 + s, r] * 2.0 ** (rho - 24), s_ref[s, r])
                    else:
                        assert e[p0 + s, r] == EXP_NONFINITE, (part, r, s)
                        assert not q[p0 + s, r].any(), (part, r, s)
        assert pl.nonfinite()
        assert int(pl.flags.item()) & 8  # OZK_FLAG_INF_SLICE (rows 1, 3, 7 lo parts)


def test_extract_i8_finite_lines_raise_no_inf_flag(ll):
    X = np.random.RandomState(3).randn(4, 6000)
    case("ozk_extract_f32_i8 finite lines: no flags")
    pl = ll.extract(X, 0, O.rho_f32(6000), 4, 1, i8=True)
    assert int(pl.flags.item()) == 0
    assert (pl.exponents().cpu().numpy() != EXP_NONFINITE).all()


# ---------------------------------------------------------------- matmul

@pytest.mark.parametrize("precision", ["high", "medium", "max"])
def test_matmul_i8_edge_rows(ozk, precision):
    """K = 8192 (INT8 planes): rows / columns whose slices overflow come out
    NaN exactly where the reference's do, for the fused 2Sum order and the
    FP64 block order; every other element is bit-exact."""
    N, K, M = 40, 8192, 36
    A, B = edge_operands(N, K, M, 81)
    nh, nl = OP.resolve_precision(precision)
    for acc, f in [("fused", O.matmul_ondevice_a4), ("host", O.matmul_ondevice_a3)]:
        case(f"matmul ondevice {precision} {acc} edge rows ({N},{K},{M})")
        C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=precision)
        ref = quiet(f, A, B, "raise", nh, nl)
        assert np.isnan(ref).any() and np.isfinite(ref).sum() > N * M // 2
        assert np.array_equal(C, ref, equal_nan=True)


@pytest.mark.parametrize("precision", ["high", "medium"])
def test_matmul_i8_inf_slice_host_order(ozk, precision):
    """A row whose only nonzero slice is all +inf (1.5 * 2^-129: 2^-c
    overflows, no zero grid value) against a column whose every slice is
    positive: the FP64 block order gives C = +inf there, which the INT8
    planes cannot carry; the call is repeated on BF16 planes."""
    N, K, M = 6, 8192, 5
    rng = np.random.RandomState(1)
    A, B = rng.randn(N, K), rng.randn(K, M)
    A[2] = 1.5 * 2.0 ** -129
    B[:, 1] = 1 + 2.0 ** -7 + 2.0 ** -14 + 2.0 ** -21 + 2.0 ** -30
    nh, nl = OP.resolve_precision(precision)
    case(f"matmul ondevice {precision} host +inf slice ({N},{K},{M})")
    C = ozk.matmul(A, B, pipeline="ondevice", accumulation="host", precision=precision)
    ref = quiet(O.matmul_ondevice_a3, A, B, "raise", nh, nl)
    assert ref[2, 1] == np.inf
    assert np.array_equal(C, ref, equal_nan=True)
    case(f"matmul ondevice {precision} fused +inf slice ({N},{K},{M})")
    C = ozk.matmul(A, B, pipeline="ondevice", accumulation="fused", precision=precision)
    ref = quiet(O.matmul_ondevice_a4, A, B, "raise", nh, nl)
    assert np.isnan(ref[2]).all()
    assert np.array_equal(C, ref, equal_nan=True)


def test_matmul_i8_tail_split_edge_rows(ozk):
    """The K-split tail (1100^2 output, 324 tiles) folds the summed pieces
    with the same NaN scales."""
    N, K, M = 1100, 8192, 1100
    A, B = edge_operands(N, K, M, 91)
    rows = np.r_[0:8, N - 40:N]
    case(f"matmul ondevice high fused tail split edge rows ({N},{K},{M})")
    C = ozk.matmul(A, B, pipeline="ondevice", precision="high")
    ref = quiet(O.matmul_ondevice_a4, A[rows], B)
    assert np.array_equal(C[rows], ref, equal_nan=True)


# ---------------------------------------------------------------- gram / residual

@pytest.mark.parametrize("precision", ["high", "max"])
def test_gram_i8_edge_columns(ozk, precision):
    """gram runs no preflight (gram.py:47-99): columns scaled by 2^-110 and
    2^110, a NaN and an Inf give NaN rows and columns of G, as in the
    reference.  8192 rows: INT8 planes."""
    rng = np.random.RandomState(17)
    A = rng.randn(8192, 40)
    A[:, 3] *= 2.0 ** -110
    A[:, 9] *= 2.0 ** 110
    A[100, 20] = np.nan
    A[5000, 33] = -np.inf
    case(f"gram ozaki {precision} edge columns (8192, 40)")
    G = ozk.gram(A, mode="ozaki", precision=precision)
    ref = quiet(O.gram_ozaki, A, precision)
    assert np.isnan(ref).any() and np.isfinite(ref).any()
    assert np.array_equal(G, ref, equal_nan=True)


def test_residual_i8_edge_rows(ozk):
    """residual at K = 8192 (slice GEMM on INT8 planes): overflowing rows of A
    and a NaN in A give NaN entries of r; a NaN in x makes all of r NaN."""
    N, K = 300, 8192
    rng = np.random.RandomState(23)
    A, x, b = rng.randn(N, K), rng.randn(K), rng.randn(N)
    A[10] *= 2.0 ** -110
    A[11] *= 2.0 ** 110
    A[12, 77] = np.nan
    case(f"residual ozaki edge rows ({N},{K})")
    r = ozk.residual(A, x, b, mode="ozaki")
    ref = quiet(O.residual_ozaki, A, x, b)
    assert np.isnan(ref[10:13]).all() and np.isfinite(ref).sum() == N - 3
    assert np.array_equal(r, ref, equal_nan=True)
    x2 = x.copy()
    x2[5] = np.nan
    case(f"residual ozaki NaN in x ({N},{K})")
    r = ozk.residual(A, x2, b, mode="ozaki")
    assert np.isnan(r).all()
    assert np.array_equal(r, quiet(O.residual_ozaki, A, x2, b), equal_nan=True)
