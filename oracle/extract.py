"""Sigma-trick slice extraction, restated in NumPy (test infrastructure only).

Restates ``ozaki_jax/extract.py`` of the reference.  The arithmetic is the
reference's: per slice, the row (or column) maximum of |residual| gives an
exponent c = floor(log2(max)) evaluated with ``np.log2`` in the working
precision (0 for an all-zero line); sigma = 0.75 * 2^(rho + c); the slice value
is v = (R + sigma) - sigma; the residual becomes R - v; the stored slice is
v * 2^-c.  Results are returned stacked: slices (n, rows, cols), exponents
(n, lines).
"""

import math

import numpy as np


def _rho(K, m1, m2, m3):
    """rho = max(ceil(m1 - (m3 - ceil(log2 max(K, 2))) / 2), m1 + 1 - m2).

    Follows extract.py:12-18 (FP64: m1=53) and extract.py:109-113 (FP32: m1=24).
    Integer arithmetic only; ceil(log2 K) for K >= 2 is (K-1).bit_length().
    """
    k = max(int(K), 2)
    clog2 = (k - 1).bit_length()
    num = 2 * m1 - m3 + clog2          # 2 * (m1 - (m3 - clog2)/2)
    gamma = -((-num) // 2)             # ceil(num / 2)
    return max(gamma, m1 + 1 - m2)


def rho_f64(K):
    """extract.py:12-18 (`_compute_rho`)."""
    return _rho(K, 53, 8, 24)


def rho_f32(K):
    """extract.py:109-113 (`_compute_rho_f32`)."""
    return _rho(K, 24, 8, 24)


def _extract_lines(X, rho, n_slices, axis, dtype, exp_int_dtype):
    """Shared body of the four extraction routines.

    axis=1 -> one exponent per row (extract.py:30, :125);
    axis=0 -> one exponent per column (extract.py:77, :166).
    """
    one = dtype(1.0)
    R = np.array(X, dtype=dtype, copy=True)
    lines = R.shape[0] if axis == 1 else R.shape[1]
    bshape = (lines, 1) if axis == 1 else (1, lines)
    slices = np.empty((n_slices,) + R.shape, dtype=np.float32)
    exps = np.empty((n_slices, lines), dtype=dtype)
    for s in range(n_slices):
        m = np.max(np.abs(R), axis=axis).astype(dtype)           # :30 / :125
        zero = m == 0                                            # :33 / :127
        c = np.floor(np.log2(np.where(zero, one, m)).astype(dtype))  # :37 / :130
        c = np.where(zero, dtype(0.0), c).astype(dtype)
        sig = (dtype(0.75) * np.ldexp(np.ones(lines, dtype=dtype),
                                      (rho + c).astype(exp_int_dtype))).astype(dtype)
        sig = sig.reshape(bshape)
        v = ((R + sig).astype(dtype) - sig).astype(dtype)          # :46 / :140
        v = np.where(zero.reshape(bshape), dtype(0.0), v).astype(dtype)
        R = (R - v).astype(dtype)                                # :52 / :142
        inv = np.ldexp(np.ones(lines, dtype=dtype),
                       (-c).astype(exp_int_dtype)).astype(dtype).reshape(bshape)
        slices[s] = (v * inv).astype(dtype).astype(np.float32)   # :57-60 / :148
        exps[s] = c
    return slices, exps, R


def extract_rows_f64(X, rho, n_slices=8, return_residual=False):
    """extract.py:21-65: FP64 row extraction; slices as float32, exps float64."""
    s, e, R = _extract_lines(np.asarray(X, np.float64), rho, n_slices, 1,
                             np.float64, np.int64)
    return (s, e, R) if return_residual else (s, e)


def extract_cols_f64(X, rho, n_slices=8):
    """extract.py:68-103: FP64 column extraction."""
    s, e, _ = _extract_lines(np.asarray(X, np.float64), rho, n_slices, 0,
                             np.float64, np.int64)
    return s, e


def extract_rows_f32(X, rho, n_slices=5, return_residual=False):
    """extract.py:116-154: FP32 row extraction; exps float32."""
    s, e, R = _extract_lines(np.asarray(X, np.float32), rho, n_slices, 1,
                             np.float32, np.int32)
    return (s, e, R) if return_residual else (s, e)


def extract_cols_f32(X, rho, n_slices=5, return_residual=False):
    """extract.py:157-191: FP32 column extraction; exps float32."""
    s, e, R = _extract_lines(np.asarray(X, np.float32), rho, n_slices, 0,
                             np.float32, np.int32)
    return (s, e, R) if return_residual else (s, e)


def ceil_log2(K):
    """ceil(log2(max(K, 2))) as used in rho (helper for tests)."""
    return int(math.ceil(math.log2(max(K, 2))))
