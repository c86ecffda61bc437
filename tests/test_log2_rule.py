"""The kernels' exponent rule c = e + (m >= T_e) (log2_thresholds.inc) equals
floor(np.log2(m)) in the working precision, as the reference computes it
(extract.py:37, :82, :130, :171).  FP32: every positive finite value.  FP64:
a window around every binade's threshold plus random samples.

Runs on whatever host executes it: on a GPU machine it re-checks that
machine's NumPy against the same table."""

import importlib.util
import re

import numpy as np
import pytest

from conftest import ROOT

CSRC = ROOT / "ozaki-jax_amd" / "csrc"


def _tables_from_inc():
    text = (CSRC / "log2_thresholds.inc").read_text()
    b32 = re.search(r"ozk_thr32_bits\[OZK_THR32_COUNT\] = \{(.*?)\};", text, re.S).group(1)
    b64 = re.search(r"ozk_thr64_bits\[OZK_THR64_COUNT\] = \{(.*?)\};", text, re.S).group(1)
    t32 = np.array([int(x.strip().rstrip("u"), 16) for x in b32.split(",") if x.strip()],
                   dtype=np.uint32).view(np.float32)
    t64 = np.array([int(x.strip().rstrip("ul"), 16) for x in b64.split(",") if x.strip()],
                   dtype=np.uint64).view(np.float64)
    return t32, t64


def test_inc_matches_generator():
    spec = importlib.util.spec_from_file_location("gen", CSRC / "gen_log2_thresholds.py")
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    assert gen.render(*gen.tables()) == (CSRC / "log2_thresholds.inc").read_text()


def test_fp32_fast_path_bound():
    """floor_log2_rn(float) returns the binade e without a table lookup when
    m is normal and its mantissa field is below kLog2FastMant32; that is
    exact iff no threshold inside its binade has a smaller mantissa field."""
    fast = int(re.search(r"kLog2FastMant32 = (0x[0-9a-fA-F]+)u;",
                         (CSRC / "sigma.h").read_text()).group(1), 16)
    t32, _ = _tables_from_inc()
    emin = int(re.search(r"OZK_THR32_EMIN \((-?\d+)\)",
                         (CSRC / "log2_thresholds.inc").read_text()).group(1))
    bits = t32.view(np.uint32).astype(np.int64)
    inside = 0
    for i, b in enumerate(bits):
        e, ex = emin + i, (b >> 23) & 0xFF
        if ex == 0xFF:
            assert b == 0x7F800000  # +inf: no threshold in this binade
        elif ex != 0 and ex - 127 == e:
            assert (b & 0x7FFFFF) >= fast, (e, hex(b))
            inside += 1
        else:
            assert e < -126  # subnormal binades always take the table
    assert inside > 200


def _binade32(u):
    ex = (u >> 23).astype(np.int64)
    mant = (u & 0x7FFFFF).astype(np.int64)
    e = ex - 127
    den = ex == 0
    if den.any():
        e[den] = np.floor(np.log2(mant[den].astype(np.float64))).astype(np.int64) - 149
    return e


def _check32(u, t32):
    m = u.view(np.float32)
    c = np.floor(np.float32(np.log2(m))).astype(np.int64)
    e = _binade32(u)
    pred = e + (m >= t32[e + 149]).astype(np.int64)
    bad = np.nonzero(pred != c)[0]
    assert bad.size == 0, (u[bad[:5]], c[bad[:5]], pred[bad[:5]])


def test_fp32_rule_near_thresholds():
    t32, _ = _tables_from_inc()
    u = []
    for e in range(-149, 128):
        top = np.float32(2.0 ** (e + 1)) if e < 127 else np.float32(np.inf)
        hi = int(np.array(top, np.float32).view(np.uint32)) if e < 127 else 0x7F800000
        u.extend(range(max(hi - 64, 1), hi))
        lo = int(np.array(np.float32(2.0 ** e) if e >= -149 else 0, np.float32).view(np.uint32))
        u.extend(range(max(lo, 1), lo + 8))
    _check32(np.unique(np.array(u, dtype=np.uint32)), t32)


@pytest.mark.slow
def test_fp32_rule_exhaustive():
    """All 2^31 - 2^23 positive finite float32 values (~45 s)."""
    t32, _ = _tables_from_inc()
    step = 1 << 24
    for start in range(1, 0x7F800000, step):
        _check32(np.arange(start, min(start + step, 0x7F800000), dtype=np.uint32), t32)


def test_fp64_rule():
    _, t64 = _tables_from_inc()
    vals = []
    for e in range(-1074, 1024):
        top = 2.0 ** (e + 1) if e < 1023 else np.inf
        x = np.float64(top) if e < 1023 else np.float64(np.finfo(np.float64).max)
        u = int(np.array(x).view(np.uint64))
        if e < 1023:
            vals.extend(range(max(u - 48, 1), u))
        else:
            vals.extend(range(u - 47, u + 1))
        lo = int(np.array(np.float64(2.0 ** e)).view(np.uint64))
        vals.extend(range(lo, lo + 4))
    rng = np.random.RandomState(0)
    vals.extend(rng.randint(1, 0x7FEFFFFFFFFFFFFF, size=200000, dtype=np.int64).tolist())
    u = np.unique(np.array(vals, dtype=np.uint64))
    u = u[u > 0]
    m = u.view(np.float64)
    c = np.floor(np.log2(m)).astype(np.int64)
    ex = (u >> np.uint64(52)).astype(np.int64)
    mant = (u & np.uint64((1 << 52) - 1)).astype(np.int64)
    e = ex - 1023
    den = ex == 0
    e[den] = np.array([int(v).bit_length() - 1 for v in mant[den]], dtype=np.int64) - 1074
    pred = e + (m >= t64[e + 1074]).astype(np.int64)
    bad = np.nonzero(pred != c)[0]
    assert bad.size == 0, (u[bad[:5]], c[bad[:5]], pred[bad[:5]])
