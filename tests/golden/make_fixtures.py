"""Writes the golden fixtures of tests/golden from the oracle (CPU only).

  log2_edges.npz     FP64 matrices whose row / column maxima (of the FP32 hi
                     part, and of the FP64 values) sit at and just below the
                     exponent-rounding thresholds of binades around 2^k, with
                     the oracle's expected slices and exponents.
  config1.json       digests of the 256x256 host-pipeline case (RandomState(0),
                     n_slices=8): slices, exponents, per-pair products and C.

Usage: python tests/golden/make_fixtures.py
"""

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

import oracle as O  # noqa: E402


def _edge_values_f32(rng, count):
    """float32 values at T_e - j ulp (j in 0..2) and at 2^(e+1) - j ulp for
    binades where floor(RN(log2)) rounds up, as float64."""
    out = []
    for k in list(range(3, 40)) + [-2] + list(range(-40, -3)):
        top = np.float32(2.0 ** k)
        for j in (1, 2, 5, 10, 11, 12, 13, 21, 22, 23):
            v = top
            for _ in range(j):
                v = np.nextafter(v, np.float32(0))
            out.append(float(v))
    rng.shuffle(out)
    return np.array(out[:count])


def _edge_values_f64(rng, count):
    out = []
    for k in list(range(3, 60)) + list(range(-60, -2)):
        top = np.float64(2.0 ** k)
        for j in (1, 2, 10, 11, 12, 21, 22, 23, 44, 45):
            out.append(float(top - j * np.spacing(np.nextafter(top, 0))))
    rng.shuffle(out)
    return np.array(out[:count])


def log2_edges():
    rng = np.random.RandomState(2024)
    rows, cols = 96, 40
    # FP32 path: each row's max is an edge value, the rest smaller
    e32 = _edge_values_f32(rng, rows)
    X32 = rng.uniform(-1, 1, (rows, cols)) * e32[:, None] * 0.5
    X32[np.arange(rows), rng.randint(0, cols, rows)] = e32 * np.where(rng.rand(rows) < 0.5, -1, 1)
    X32[5] = 0.0
    e64 = _edge_values_f64(rng, rows)
    X64 = rng.uniform(-1, 1, (rows, cols)) * e64[:, None] * 0.5
    X64[np.arange(rows), rng.randint(0, cols, rows)] = e64
    X64[7] = 0.0
    out = {"X32": X32, "X64": X64}
    rho32 = O.rho_f32(cols)
    hi, lo = O.split_hi_lo(X32)
    out["rows32_s"], out["rows32_e"] = O.extract_rows_f32(hi, rho32, 4)
    out["rows32_lo_s"], out["rows32_lo_e"] = O.extract_rows_f32(lo, rho32, 1)
    rho32c = O.rho_f32(rows)
    hiT, loT = O.split_hi_lo(X32.T.copy())
    out["cols32_s"], out["cols32_e"] = O.extract_cols_f32(hiT, rho32c, 4)
    rho64 = O.rho_f64(cols)
    out["rows64_s"], out["rows64_e"] = O.extract_rows_f64(X64, rho64, 8)
    out["rho32"], out["rho32c"], out["rho64"] = rho32, rho32c, rho64
    np.savez_compressed(HERE / "log2_edges.npz", **out)


def _digest(a):
    a = np.ascontiguousarray(a)
    return hashlib.sha256(a.tobytes()).hexdigest() + f":{a.dtype}:{a.shape}"


def config1():
    rs = np.random.RandomState(0)
    A = rs.randn(256, 256)
    B = rs.randn(256, 256)
    rho = O.rho_f64(256)
    a, ae, b, be = O.host_slices(A, B, rho, 8)
    sched = O.host_schedule(8)
    P = O.slice_products(a, b, sched)
    C1 = O.accumulate_a1(P, sched, ae, be)
    C2 = O.accumulate_a2(P, sched, ae, be)
    assert np.array_equal(C1, O.matmul_numpy(A, B))
    doc = {
        "case": "RandomState(0): A = randn(256,256), B = randn(256,256); "
                "matmul_numpy(A, B, n_slices=8, pipeline='host')",
        "rho64": rho,
        "a_slices": _digest(a), "a_exps": _digest(ae.astype(np.int32)),
        "b_slices_cols": _digest(b), "b_exps": _digest(be.astype(np.int32)),
        "products": _digest(P), "C_numpy_order": _digest(C1),
        "C_jax_order": _digest(C2),
        "C_row0_first8": C1[0, :8].tolist(),
    }
    (HERE / "config1.json").write_text(json.dumps(doc, indent=1) + "\n")


if __name__ == "__main__":
    log2_edges()
    config1()
