"""The short form of the FP32 slice step that the extraction and residual
kernels use where it applies (fast_step in ozaki-jax_amd/csrc/sigma.h),
checked against the plain sigma form of the oracle (oracle/extract.py
`_extract_lines`, reference extract.py:124-152) on the CPU:

  plain: v = (R + sigma) - sigma, sigma = 0.75 * 2^(rho + c); R' = R - v;
         slice = v * 2^-c
  short: q = rint(R * 2^(24 - rho - c)); R' = fma(-q, 2^(rho + c - 24), R);
         slice = q * 2^(rho - 24)

with c = floor(log2 max|R|) from the oracle.  fma is evaluated exactly in
float64 and rounded once to float32.  The INT8 byte q + offset is read from
the low byte of q + 1.5 * 2^23 + offset, as the kernels pack it."""

import numpy as np
import pytest

import oracle as O

F = np.float32


def short_form(X, rho, n):
    R = np.array(X, dtype=F)
    sl, ex, qs = [], [], []
    for _ in range(n):
        m = np.max(np.abs(R), axis=1)
        zero = m == 0
        c = np.floor(np.log2(np.where(zero, F(1), m)).astype(F))
        c = np.where(zero, F(0), c).astype(np.int32)
        e = (rho + c - 24)[:, None]
        # the kernels' condition for the short form; other lines take the plain one
        ok = (~zero[:, None]) & (np.abs(e) <= 100)
        short_lines[0] += int(ok.sum())
        ee = np.where(ok, e, 0)
        s = np.ldexp(F(1), -ee).astype(F)
        u = np.ldexp(F(1), ee).astype(F)
        q = np.rint((R * s).astype(F)).astype(F)
        Rs = (R.astype(np.float64) - q.astype(np.float64) * u.astype(np.float64)).astype(F)
        sig = (F(0.75) * np.ldexp(F(1), rho + c)).astype(F)[:, None]
        v = ((R + sig).astype(F) - sig).astype(F)
        v = np.where(zero[:, None], F(0), v).astype(F)
        inv = np.ldexp(F(1), -c).astype(F)[:, None]
        qp = ((v * inv).astype(F) * np.ldexp(F(1), 24 - rho)).astype(F)
        q = np.where(ok, q, qp).astype(F)
        R = np.where(ok, Rs, (R - v).astype(F)).astype(F)
        sl.append((q * np.ldexp(F(1), rho - 24)).astype(F) + F(0))
        ex.append(c)
        qs.append(q)
    return np.array(sl), np.array(ex), R, np.array(qs)


short_lines = [0]


def lines(kind, seed):
    rng = np.random.RandomState(seed)
    if kind == "randn":
        X = rng.randn(64, 257)
        X[::7] = 0.0  # zero lines: plain form, zero slices
        X[1::7, 5:] = 0.0  # lines whose residual vanishes after a few slices
    elif kind == "wide":
        X = (rng.rand(64, 257) - 0.5) * np.exp(4.0 * rng.randn(64, 257))
    elif kind == "ties":
        # elements on half-grid points of the first slice: R * 2^(24 - rho - c) = k + 1/2
        X = (rng.randint(-60, 60, size=(64, 257)) + 0.5) * 2.0 ** (-5)
        X[:, 0] = 1.96875
    elif kind == "integers":
        X = rng.randint(-1000, 1000, size=(64, 257)).astype(np.float64)
    else:
        X = rng.randn(64, 257) * 2.0 ** rng.randint(-90, 90, size=(64, 1))
    return X.astype(F)


@pytest.mark.parametrize("kind", ["randn", "wide", "ties", "integers", "scaled"])
@pytest.mark.parametrize("rho", [17, 18, 19, 21, 24])
def test_short_form_matches_the_plain_form(kind, rho):
    X = lines(kind, rho)
    ref_s, ref_e, ref_R = O.extract.__dict__["_extract_lines"](X, rho, 5, 1, np.float32, np.int32)
    short_lines[0] = 0
    s, e, R, q = short_form(X, rho, 5)
    assert short_lines[0] >= (4 if kind == "scaled" else 5) * X.shape[0] // 5
    assert np.array_equal(e, ref_e.astype(np.int32))
    assert np.array_equal(s.view(np.uint32), ref_s.view(np.uint32))  # +0 for zero slices
    assert np.array_equal(R, ref_R)  # values (a zero residual may differ in sign)
    # INT8 bytes where the grid holds them (rho >= 19): the low byte of
    # q + 1.5 * 2^23 + offset is q + offset in two's complement
    if rho >= 19:
        off = (1 << (25 - rho)) - 1
        carrier = (q + F(12582912.0 + off)).astype(F)
        byte = (carrier.view(np.uint32) & 0xFF).astype(np.uint8).view(np.int8)
        assert np.all(np.abs(q) <= 2 ** (25 - rho))
        assert np.array_equal(byte.astype(np.int32), (q.astype(np.int32) + off).astype(np.int8))


def test_ties_round_to_even():
    # R * 2^(24 - rho - c) = k + 1/2 for every k in [-64, 63]: both forms send it to the even neighbour
    rho = 19
    k = np.arange(-64, 64)
    X = np.zeros((1, k.size + 1), F)
    X[0, :-1] = (k + 0.5) * 2.0 ** -5
    X[0, -1] = 1.984375  # m in [1, 2): c = 0, grid 2^(rho + c - 24) = 2^-5
    ref_s, _, _ = O.extract.__dict__["_extract_lines"](X, rho, 1, 1, np.float32, np.int32)
    s, _, _, q = short_form(X, rho, 1)
    assert np.array_equal(s, ref_s)
    assert np.all(q[0, 0, :-1] % 2 == 0)
