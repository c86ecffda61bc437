"""FP32 column extraction without a transposed copy (columns of up to 4096
rows held whole by one workgroup; 4097 to 65536 rows cut into 512-row runs
held by the workgroups of a gang, which combine their column maxima through
the workspace), against the oracle's column extraction (extract.py:157-191,
:21-103 for FP64).

Lengths straddle the runs (gangs of 2 to 128 workgroups) and the 65536-row
limit (65537 rows go through the FP64 transpose, as FP64 extraction always
does); column counts that are not a multiple of the 16-column panel, and
odd counts (an odd leading dimension takes the element-wise loads), leave
partial panels.  Bar: bit-exact slices and exponents, zero padding.
"""

import sys

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

EXP_NONFINITE = -2 ** 31


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ll(ozk):
    from ozaki_jax_amd import lowlevel
    return lowlevel


def gen(kind, shape, seed):
    rng = np.random.RandomState(seed)
    if kind == "wide":
        return (rng.rand(*shape) - 0.5) * np.exp(4.0 * rng.randn(*shape))
    X = rng.randn(*shape)
    if kind == "zerocols":
        X[:, ::3] = 0.0
        X[: shape[0] // 2, 1 % shape[1]] = 0.0
    return X


def to_np(t):
    return t.cpu().numpy()


def check_padding(pl, rows, cols):
    """Padding holds zero slices; INT8 line sums are those of the counts."""
    g = to_np(pl.counts() if pl.i8 else pl.grid())
    assert not g[:, :, rows:].any() and not g[:, cols:, :].any(), "padding"
    if pl.i8:
        assert np.array_equal(to_np(pl.sums), g.astype(np.int64).sum(axis=2)), "line sums"


LENGTHS = [1, 100, 511, 513, 1025, 2049, 4097, 5000, 8192, 8193]
COLS = [1, 33, 130]


@pytest.mark.parametrize("length", LENGTHS)
@pytest.mark.parametrize("cols", COLS)
def test_panel_f32_bf16(ll, length, cols):
    X = gen("wide" if cols != 33 else "zerocols", (length, cols), length + cols)
    rho = O.rho_f32(length)
    hi, lo = O.split_hi_lo(X)
    for n0, n1 in ((4, 1), (2, 3)):
        case(f"ozk_extract_f32 panel ({length}, {cols}) ({n0},{n1}) rho={rho}")
        pl = ll.extract(X, 1, rho, n0, n1)
        sh, eh = O.extract_cols_f32(hi, rho, n0)
        sl, el = O.extract_cols_f32(lo, rho, n1)
        ref = np.concatenate([sh, sl]).transpose(0, 2, 1)
        assert np.array_equal(to_np(pl.values()), ref), "slices"
        assert np.array_equal(to_np(pl.exponents()),
                              np.concatenate([eh, el]).astype(np.int32)), "exponents"
        assert not pl.nonfinite()
        check_padding(pl, length, cols)


@pytest.mark.parametrize("length", LENGTHS)
@pytest.mark.parametrize("cols", COLS)
def test_panel_f32_i8(ll, length, cols):
    X = gen("zerocols" if cols == 130 else "randn", (length, cols), 3 * length + cols)
    rho = max(19, O.rho_f32(length))
    hi, lo = O.split_hi_lo(X)
    case(f"ozk_extract_f32_i8 panel ({length}, {cols}) rho={rho}")
    pl = ll.extract(X, 1, rho, 4, 1, i8=True)
    sh, eh = O.extract_cols_f32(hi, rho, 4)
    sl, el = O.extract_cols_f32(lo, rho, 1)
    ref = np.concatenate([sh, sl]).transpose(0, 2, 1).astype(np.float64) * 2.0 ** (24 - rho)
    assert np.all(np.abs(ref) <= 64) and np.array_equal(ref, np.round(ref))
    q = to_np(pl.counts())[:, :cols, :length]
    assert np.array_equal(q, ref), "int8 slices"
    assert np.array_equal(to_np(pl.exponents()),
                          np.concatenate([eh, el]).astype(np.int32)), "exponents"
    check_padding(pl, length, cols)


LONG = [8193, 16385, 32768, 40000, 65536, 65537]


@pytest.mark.parametrize("length", LONG)
def test_gang_long_columns(ll, length):
    """Columns of 16 to 128 runs (gangs whose members combine their keys in
    batches) and, past 65536 rows, the transposed copy: both plane formats,
    33 columns (a partial panel), wide-range and zero columns."""
    X = gen("wide", (length, 33), 5 * length)
    X[:, 7] = 0.0
    hi, lo = O.split_hi_lo(X)
    for i8 in (False, True):
        rho = max(19, O.rho_f32(length)) if i8 else O.rho_f32(length)
        case(f"ozk_extract_f32 gang ({length}, 33) i8={i8} rho={rho}")
        pl = ll.extract(X, 1, rho, 4, 1, i8=i8)
        sh, eh = O.extract_cols_f32(hi, rho, 4)
        sl, el = O.extract_cols_f32(lo, rho, 1)
        ref = np.concatenate([sh, sl]).transpose(0, 2, 1)
        assert np.array_equal(to_np(pl.values()), ref), "slices"
        assert np.array_equal(to_np(pl.exponents()),
                              np.concatenate([eh, el]).astype(np.int32)), "exponents"
        assert not pl.nonfinite()
        check_padding(pl, length, 33)


@pytest.mark.parametrize("length", [4097, 8192, 32768])
@pytest.mark.parametrize("kind", ["integers", "spiky", "binade"])
def test_panel_f32_candidates_missed(ll, length, kind):
    """Columns whose later exponents are not the two candidates the gangs'
    second round sends keys for (residuals that vanish, or that fall more
    than one binade below the bound): those columns settle their slices one
    round at a time, bit-exact, on both plane formats."""
    rng = np.random.RandomState(length + len(kind))
    if kind == "integers":      # few significant bits: residuals reach zero
        X = rng.randint(-300, 300, size=(length, 40)).astype(np.float64)
    elif kind == "spiky":       # one large element per column, the rest tiny
        X = rng.randn(length, 40) * 1e-6
        X[rng.randint(0, length, 40), np.arange(40)] = 1e3
    else:                       # every element in [1, 2): exponent steps of the bound
        X = 1.0 + rng.rand(length, 40)
    hi, lo = O.split_hi_lo(X)
    for i8 in (False, True):
        rho = max(19, O.rho_f32(length)) if i8 else O.rho_f32(length)
        case(f"ozk_extract_f32 gang {kind} ({length}, 40) i8={i8} rho={rho}")
        pl = ll.extract(X, 1, rho, 4, 1, i8=i8)
        sh, eh = O.extract_cols_f32(hi, rho, 4)
        sl, el = O.extract_cols_f32(lo, rho, 1)
        ref = np.concatenate([sh, sl]).transpose(0, 2, 1)
        assert np.array_equal(to_np(pl.values()), ref), "slices"
        assert np.array_equal(to_np(pl.exponents()),
                              np.concatenate([eh, el]).astype(np.int32)), "exponents"
        check_padding(pl, length, 40)


@pytest.mark.parametrize("length", [40000, 65536])
@pytest.mark.parametrize("kind", ["wide", "integers", "spiky", "binade"])
def test_row_gang_rounds(ll, length, kind):
    """Rows of 32769 to 262144 elements, held by gangs of 16384-element runs
    that settle one slice per exchange round: wide-range rows, rows whose
    residuals vanish (integers), one large element among tiny ones (spiky),
    every element in [1, 2) (binade), and a zero row; both plane formats,
    bit-exact, with the members' INT8 line sums added up."""
    rng = np.random.RandomState(length + 7 * len(kind))
    shape = (13, length)
    if kind == "wide":
        X = gen("wide", shape, length)
    elif kind == "integers":
        X = rng.randint(-300, 300, size=shape).astype(np.float64)
    elif kind == "spiky":
        X = rng.randn(*shape) * 1e-6
        X[np.arange(13), rng.randint(0, length, 13)] = 1e3
    else:
        X = 1.0 + rng.rand(*shape)
    X[4] = 0.0
    hi, lo = O.split_hi_lo(X)
    for i8 in (False, True):
        rho = max(19, O.rho_f32(length)) if i8 else O.rho_f32(length)
        case(f"ozk_extract_f32 row gang {kind} (13, {length}) i8={i8} rho={rho}")
        pl = ll.extract(X, 0, rho, 4, 1, i8=i8)
        sh, eh = O.extract_rows_f32(hi, rho, 4)
        sl, el = O.extract_rows_f32(lo, rho, 1)
        assert np.array_equal(to_np(pl.values()), np.concatenate([sh, sl])), "slices"
        assert np.array_equal(to_np(pl.exponents()),
                              np.concatenate([eh, el]).astype(np.int32)), "exponents"
        check_padding(pl, length, 13)


@pytest.mark.parametrize("length", [1024, 2049, 4097, 8192])
def test_panel_f64(ll, length):
    X = gen("wide", (length, 35), 11 + length)
    rho = O.rho_f64(length)
    case(f"ozk_extract_f64 panel ({length}, 35) rho={rho}")
    pl = ll.extract(X, 1, rho, 8, f64=True)
    s, e = O.extract_cols_f64(X, rho, 8)
    assert np.array_equal(to_np(pl.values()), s.transpose(0, 2, 1)), "slices"
    assert np.array_equal(to_np(pl.exponents()), e.astype(np.int32)), "exponents"
    check_padding(pl, length, 35)


@pytest.mark.parametrize("length", [2000, 8192, 40000])
def test_panel_nonfinite_columns(ll, length):
    """A NaN, an Inf and a 2^110-scaled column: the flag word reports the
    non-finite input; on INT8 planes the NaN and Inf columns carry the
    non-finite exponent in every plane, the scaled column in its hi planes
    (sigma overflows; its lo part, near 2^86, does not), and the other
    columns keep the oracle's slices."""
    rng = np.random.RandomState(length)
    X = rng.randn(length, 20)
    X[length - 1, 3] = np.nan
    X[7, 8] = np.inf
    X[:, 12] *= 2.0 ** 110
    rho = max(19, O.rho_f32(length))
    case(f"ozk_extract_f32 panel non-finite ({length}, 20)")
    assert ll.extract(X, 1, rho, 4, 1).nonfinite()
    case(f"ozk_extract_f32_i8 panel non-finite ({length}, 20)")
    pl = ll.extract(X, 1, rho, 4, 1, i8=True)
    assert pl.nonfinite()
    e = to_np(pl.exponents())
    assert np.all(e[:, [3, 8]] == EXP_NONFINITE) and np.all(e[:4, 12] == EXP_NONFINITE)
    good = [c for c in range(20) if c not in (3, 8, 12)]
    hi, lo = O.split_hi_lo(X[:, good])
    sh, eh = O.extract_cols_f32(hi, rho, 4)
    sl, el = O.extract_cols_f32(lo, rho, 1)
    ref = np.concatenate([sh, sl]).transpose(0, 2, 1) * 2.0 ** (24 - rho)
    q = to_np(pl.counts())[:, good, :length]
    assert np.array_equal(q, ref), "int8 slices"
    check_padding(pl, length, 20)
    assert np.array_equal(e[:, good], np.concatenate([eh, el]).astype(np.int32))
