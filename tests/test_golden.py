"""The committed golden fixtures (tests/golden) equal what the oracle computes
on this machine: pins the oracle's NumPy-dependent behaviour (np.log2 near
powers of two, sgemm of exact integers) across hosts."""

import hashlib
import json

import numpy as np

import oracle as O


def _digest(a):
    a = np.ascontiguousarray(a)
    return hashlib.sha256(a.tobytes()).hexdigest() + f":{a.dtype}:{a.shape}"


def test_log2_edges_fixture(golden_dir):
    d = np.load(golden_dir / "log2_edges.npz")
    X32, X64 = d["X32"], d["X64"]
    hi, lo = O.split_hi_lo(X32)
    s, e = O.extract_rows_f32(hi, int(d["rho32"]), 4)
    assert np.array_equal(s, d["rows32_s"]) and np.array_equal(e, d["rows32_e"])
    s, e = O.extract_rows_f32(lo, int(d["rho32"]), 1)
    assert np.array_equal(s, d["rows32_lo_s"]) and np.array_equal(e, d["rows32_lo_e"])
    hiT, _ = O.split_hi_lo(X32.T.copy())
    s, e = O.extract_cols_f32(hiT, int(d["rho32c"]), 4)
    assert np.array_equal(s, d["cols32_s"]) and np.array_equal(e, d["cols32_e"])
    s, e = O.extract_rows_f64(X64, int(d["rho64"]), 8)
    assert np.array_equal(s, d["rows64_s"]) and np.array_equal(e, d["rows64_e"])


def test_config1_fixture(golden_dir):
    doc = json.loads((golden_dir / "config1.json").read_text())
    rs = np.random.RandomState(0)
    A, B = rs.randn(256, 256), rs.randn(256, 256)
    a, ae, b, be = O.host_slices(A, B, doc["rho64"], 8)
    sched = O.host_schedule(8)
    P = O.slice_products(a, b, sched)
    assert _digest(a) == doc["a_slices"] and _digest(b) == doc["b_slices_cols"]
    assert _digest(ae.astype(np.int32)) == doc["a_exps"]
    assert _digest(be.astype(np.int32)) == doc["b_exps"]
    assert _digest(P) == doc["products"]
    assert _digest(O.matmul_numpy(A, B)) == doc["C_numpy_order"]
