"""Parity of the HIP path (through the C ABI) with the oracle.

Bar: bit-exact slices, exponents, per-pair products and outputs (values
compared with np.array_equal, so +0 == -0) against the oracle restating the
same accumulation order; the 2-ulp scaled bound |C - C_ref| <= 2^-51 (|A||B|)
is asserted as well.  Sizes keep the oracle to seconds.
"""

import json
import sys

import numpy as np
import pytest

import oracle as O
from oracle import pipeline as OP

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def rel_err(a, r):
    d = np.linalg.norm(r)
    return 0.0 if d == 0 else float(np.linalg.norm(a - r) / d)


def gen(kind, shape, seed):
    rng = np.random.RandomState(seed)
    if kind == "randn":
        return rng.randn(*shape)
    if kind == "wide":      # (U - 0.5) * exp(4 N)
        return (rng.rand(*shape) - 0.5) * np.exp(4.0 * rng.randn(*shape))
    if kind == "wide2":
        return (rng.rand(*shape) - 0.5) * np.exp(2.0 * rng.randn(*shape))
    if kind == "scaled":
        return rng.randn(*shape) * 10.0 ** rng.uniform(-10, 30)
    if kind == "zerorows":
        X = rng.randn(*shape)
        X[::3] = 0.0
        if X.shape[1] > 2:
            X[:, 1] = 0.0
        return X
    raise ValueError(kind)


@pytest.fixture(scope="module")
def ll(ozk):
    from ozaki_jax_amd import lowlevel
    return lowlevel


def to_np(t):
    return t.cpu().numpy()


# ---------------------------------------------------------------- layout

def test_mfma_output_layout(ll):
    case("probe_mfma_layout 32x32x16 / 16x16x32 bf16, 16x16x64 i8")
    out, out16, out8, out8_32 = ll.probe_mfma_layout()
    for lane in range(64):
        for r in range(16):
            row = 8 * (r // 4) + 4 * (lane // 32) + (r % 4)
            col = lane % 32
            assert out[lane, r] == row + 64 * col, (lane, r, out[lane, r])
            assert out8_32[lane, r] == row + 64 * col, (lane, r, out8_32[lane, r])
        for r in range(4):
            row = 4 * (lane // 16) + r
            col = lane % 16
            assert out16[lane, r] == row + 64 * col, (lane, r, out16[lane, r])
            assert out8[lane, r] == row + 16 * col, (lane, r, out8[lane, r])


# ---------------------------------------------------------------- extraction

EXTRACT_SHAPES = [(1, 1), (3, 5), (64, 64), (130, 257), (77, 1000), (5, 4100), (3, 9000)]


@pytest.mark.parametrize("kind", ["randn", "wide", "scaled", "zerorows"])
@pytest.mark.parametrize("shape", EXTRACT_SHAPES)
def test_extract_f32_rows_and_cols(ll, kind, shape):
    X = gen(kind, shape, 100 + shape[0])
    for by_cols in (0, 1):
        lines, length = (shape[1], shape[0]) if by_cols else shape
        rho = O.rho_f32(length)
        case(f"ozk_extract_f32 {kind} {shape} by_cols={by_cols} rho={rho}")
        pl = ll.extract(X, by_cols, rho, 4, 1)
        v, e = to_np(pl.values()), to_np(pl.exponents())
        hi, lo = O.split_hi_lo(X)
        if by_cols:
            sh, eh = O.extract_cols_f32(hi, rho, 4)
            sl, el = O.extract_cols_f32(lo, rho, 1)
            sh, sl = sh.transpose(0, 2, 1), sl.transpose(0, 2, 1)
        else:
            sh, eh = O.extract_rows_f32(hi, rho, 4)
            sl, el = O.extract_rows_f32(lo, rho, 1)
        ref = np.concatenate([sh, sl])
        assert np.array_equal(v, ref), "slices"
        # bit patterns too: the oracle's zero slices are +0, and so are the planes'
        assert np.array_equal(v.view(np.uint32), ref.astype(np.float32).view(np.uint32)), "bits"
        assert np.array_equal(e, np.concatenate([eh, el]).astype(np.int32)), "exponents"
        assert not pl.nonfinite()


@pytest.mark.parametrize("shape", [(1, 1), (40, 30), (130, 257), (9, 5000), (2, 17000)])
def test_extract_f64_rows_and_cols(ll, shape):
    X = gen("wide", shape, 7 + shape[1])
    for by_cols in (0, 1):
        length = shape[0] if by_cols else shape[1]
        rho = O.rho_f64(length)
        case(f"ozk_extract_f64 {shape} by_cols={by_cols} rho={rho}")
        pl = ll.extract(X, by_cols, rho, 8, f64=True)
        v, e = to_np(pl.values()), to_np(pl.exponents())
        if by_cols:
            s, ee = O.extract_cols_f64(X, rho, 8)
            s = s.transpose(0, 2, 1)
        else:
            s, ee = O.extract_rows_f64(X, rho, 8)
        assert np.array_equal(v, s) and np.array_equal(e, ee.astype(np.int32))


# Lines longer than one workgroup holds in registers: up to 256 Ki elements
# (FP32 path) a line is held by 3 to 16 workgroups that exchange their
# per-slice maxima; longer lines stream.  (n0, n1) = (2, 3) runs more lo
# slices than hi slices; lengths that are not a multiple of 4 take the
# element-wise loads; 33000 is the shortest such line (3 workgroups),
# 262144 the longest (16), 262145 streams.
LONG_CASES = [("wide2", (3, 40000), 4, 1, False), ("zerorows", (3, 40000), 4, 1, False),
              ("wide2", (2, 65536), 4, 1, False), ("wide2", (2, 70000), 4, 1, False),
              ("wide2", (3, 40000), 2, 3, False), ("randn", (3, 40000), 4, 1, True),
              ("wide2", (2, 65536), 5, 4, True), ("wide2", (3, 40001), 4, 1, False),
              ("wide2", (2, 49998), 3, 1, True), ("wide2", (2, 65533), 4, 2, False),
              ("randn", (70, 33000), 3, 1, False), ("wide2", (2, 131072), 4, 1, True),
              ("zerorows", (3, 100003), 4, 1, False), ("wide2", (1, 262144), 4, 1, False),
              ("wide2", (1, 262145), 4, 1, False)]


@pytest.mark.parametrize("kind,shape,n0,n1,i8", LONG_CASES)
def test_extract_long_lines(ll, kind, shape, n0, n1, i8):
    X = gen(kind, shape, 5 + shape[1])
    rho = O.rho_f32(shape[1])
    hi, lo = O.split_hi_lo(X)
    sh, eh = O.extract_rows_f32(hi, rho, n0)
    sl, el = O.extract_rows_f32(lo, rho, n1)
    ref = np.concatenate([sh, sl])
    for by_cols in (0, 1):
        case(f"ozk_extract_f32 long lines {kind} {shape} ({n0},{n1}) i8={i8} by_cols={by_cols}")
        pl = ll.extract(X.T.copy() if by_cols else X, by_cols, rho, n0, n1, i8=i8)
        assert np.array_equal(to_np(pl.values()), ref), "slices"
        assert np.array_equal(to_np(pl.exponents()),
                              np.concatenate([eh, el]).astype(np.int32)), "exponents"
        g = to_np(pl.counts() if i8 else pl.grid())
        assert not g[:, :, shape[1]:].any() and not g[:, shape[0]:, :].any(), "padding"
        if i8:
            assert np.array_equal(to_np(pl.sums), g.astype(np.int64).sum(axis=2)), "line sums"


def test_extract_log2_edge_fixture(ll, golden_dir):
    d = np.load(golden_dir / "log2_edges.npz")
    case("log2 edge fixture: f32 rows / cols, f64 rows")
    pl = ll.extract(d["X32"], 0, int(d["rho32"]), 4, 1)
    v, e = to_np(pl.values()), to_np(pl.exponents())
    assert np.array_equal(v[:4], d["rows32_s"]) and np.array_equal(e[:4], d["rows32_e"])
    assert np.array_equal(v[4:], d["rows32_lo_s"]) and np.array_equal(e[4:], d["rows32_lo_e"])
    pl = ll.extract(d["X32"].T.copy(), 1, int(d["rho32c"]), 4, 1)
    v, e = to_np(pl.values()), to_np(pl.exponents())
    assert np.array_equal(v[:4], d["cols32_s"].transpose(0, 2, 1))
    assert np.array_equal(e[:4], d["cols32_e"])
    pl = ll.extract(d["X64"], 0, int(d["rho64"]), 8, f64=True)
    assert np.array_equal(to_np(pl.values()), d["rows64_s"])
    assert np.array_equal(to_np(pl.exponents()), d["rows64_e"].astype(np.int32))


def test_extract_nonfinite_flag(ll):
    X = np.ones((5, 7))
    X[2, 3] = np.inf
    case("nonfinite flag (inf)")
    assert ll.extract(X, 0, 17, 4, 1).nonfinite()
    X[2, 3] = np.nan
    case("nonfinite flag (nan) by cols")
    assert ll.extract(X, 1, 17, 4, 1).nonfinite()


@pytest.mark.parametrize("length", [40000, 40001, 200000])
def test_extract_nonfinite_flag_long_lines(ll, length):
    """The long-line kernels (both load forms) raise the flag too, and only
    when a line holds a non-finite element."""
    X = np.ones((3, length))
    rho = O.rho_f32(length)
    case(f"nonfinite flag long lines {length}: finite")
    assert not ll.extract(X, 0, rho, 4, 1).nonfinite()
    X[2, length - 1] = np.inf
    case(f"nonfinite flag long lines {length}: inf last element")
    assert ll.extract(X, 0, rho, 4, 1).nonfinite()
    X[2, length - 1] = 1.0
    X[0, 1] = np.nan
    case(f"nonfinite flag long lines {length}: nan")
    assert ll.extract(X, 0, rho, 4, 1).nonfinite()


# INT8 planes: q = slice * 2^(24 - rho), exact for rho >= 19.  Lines of
# length > 4096 give rho >= 19 by themselves; shorter ones are run with an
# explicit rho in [19, 24] (any rho is a valid extraction grid).
I8_CASES = [((3, 5000), None), ((130, 4200), None), ((2, 9000), None), ((3, 16384), None),
            ((2, 20000), None), ((64, 64), 19), ((77, 300), 21), ((5, 33), 24), ((1, 1), 19)]


@pytest.mark.parametrize("kind", ["randn", "wide", "zerorows"])
@pytest.mark.parametrize("shape,rho_fixed", I8_CASES)
def test_extract_f32_i8_rows_and_cols(ll, kind, shape, rho_fixed):
    X = gen(kind, shape, 200 + shape[1])
    hi, lo = O.split_hi_lo(X)
    for by_cols in (0, 1):
        Xi = X.T.copy() if by_cols else X
        rho = rho_fixed or O.rho_f32(shape[1])
        case(f"ozk_extract_f32_i8 {kind} {shape} by_cols={by_cols} rho={rho}")
        pl = ll.extract(Xi, by_cols, rho, 4, 1, i8=True)
        sh, eh = O.extract_rows_f32(hi, rho, 4)
        sl, el = O.extract_rows_f32(lo, rho, 1)
        ref = np.concatenate([sh, sl]).astype(np.float64) * 2.0 ** (24 - rho)
        assert np.all(np.abs(ref) <= 64) and np.array_equal(ref, np.round(ref))
        g = to_np(pl.counts())
        assert np.array_equal(g[:, :shape[0], :shape[1]], ref), "int8 slices"
        assert np.array_equal(to_np(pl.exponents()),
                              np.concatenate([eh, el]).astype(np.int32)), "exponents"
        # padding holds zero slices (the GEMM reads it); the line sums are
        # those of the counts, padding lines included
        assert not g[:, :, shape[1]:].any() and not g[:, shape[0]:, :].any()
        assert np.array_equal(to_np(pl.sums), g.astype(np.int64).sum(axis=2)), "line sums"


def test_extract_i8_rejects_coarse_grid(ll):
    case("ozk_extract_f32_i8 rho=18 -> unsupported")
    with pytest.raises(NotImplementedError, match="19 <= rho"):
        ll.extract(np.ones((4, 4)), 0, 18, 4, 1, i8=True)


# ---------------------------------------------------------------- products

# (2, 3), (1, 2), (2, 1), (1, 1): one-sweep custom schedules on the
# all-pairs kernel; (4, 2), (1, 5): two sweeps of it; (5, 1): three;
# (6, 1), (1, 6), (7, 6), (8, 8): rectangle sweeps (4, 3, 7 and 12 of them;
# (6, 1), (7, 6) and (8, 8) cut blocks between groups); (9, 1): the
# pairwise kernel.  Host schedules of 1 to 9 slices run on the all-pairs
# kernel in sweeps over groups of A planes (one sweep up to 5 slices, two
# for 6 and 7, three for 8, four for 9); 10 slices on the pairwise kernel.
# Per-pair products of the rectangle schedules come from the pairwise
# kernel.
SCHEDULES = [("ondevice", 4, 1), ("ondevice", 3, 1), ("ondevice", 5, 4),
             ("ondevice", 2, 3), ("ondevice", 1, 2), ("ondevice", 2, 1),
             ("ondevice", 1, 1), ("ondevice", 4, 2), ("ondevice", 5, 1), ("ondevice", 1, 5),
             ("ondevice", 6, 1), ("ondevice", 1, 6), ("ondevice", 7, 6), ("ondevice", 8, 8),
             ("ondevice", 9, 1), ("host", 1, 0), ("host", 4, 0), ("host", 5, 0),
             ("host", 6, 0), ("host", 7, 0), ("host", 8, 0), ("host", 9, 0), ("host", 10, 0)]


def _slices(ll, A, B, pipe, nh, nl):
    K = A.shape[1]
    if pipe == "host":
        rho = O.rho_f64(K)
        a = ll.extract(A, 0, rho, nh, f64=True)
        b = ll.extract(B, 1, rho, nh, f64=True)
        oa, oae, ob, obe = O.host_slices(A, B, rho, nh)
        sched = O.host_schedule(nh)
        code = ll.PIPE_HOST
    else:
        rho = O.rho_f32(K)
        a = ll.extract(A, 0, rho, nh, nl)
        b = ll.extract(B, 1, rho, nh, nl)
        oa, oae, ob, obe = O.ondevice_slices(A, B, rho, nh, nl)
        sched = O.ondevice_schedule(nh, nl)
        code = ll.PIPE_ONDEVICE
    return a, b, (oa, oae, ob, obe), sched, code


@pytest.mark.parametrize("pipe,nh,nl", SCHEDULES)
@pytest.mark.parametrize("shape", [(96, 70, 160), (64, 64, 64), (1, 33, 1), (130, 257, 67)])
def test_slice_products_bit_exact(ll, pipe, nh, nl, shape):
    N, K, M = shape
    if pipe == "host" and K > 1024:
        pytest.skip("host schedule needs K <= 1024")
    A, B = gen("randn", (N, K), 1), gen("wide2", (K, M), 2)
    a, b, (oa, oae, ob, obe), sched, code = _slices(ll, A, B, pipe, nh, nl)
    case(f"ozk_slice_products {pipe} ({nh},{nl}) N,K,M={shape}")
    P = to_np(ll.slice_products(a, b, code, nh, nl))
    Pref = O.slice_products(oa, ob, sched)
    assert OP.products_exact_certificate(
        oa, ob, sched, 2.0 ** (O.rho_f32(K) - 24 if pipe != "host" else O.rho_f64(K) - 53),
        2.0 ** (O.rho_f32(K) - 24 if pipe != "host" else O.rho_f64(K) - 53))
    assert np.array_equal(P, Pref)


I8_SHAPES = [((96, 5000, 160), None), ((2, 8192, 3), None), ((130, 4100, 67), None),
             ((64, 64, 64), 19), ((96, 70, 160), 20), ((1, 33, 1), 24)]


def _slices_i8(ll, A, B, nh, nl, rho_fixed):
    rho = rho_fixed or O.rho_f32(A.shape[1])
    a = ll.extract(A, 0, rho, nh, nl, i8=True)
    b = ll.extract(B, 1, rho, nh, nl, i8=True)
    return a, b, O.ondevice_slices(A, B, rho, nh, nl), O.ondevice_schedule(nh, nl), rho


@pytest.mark.parametrize("nh,nl", [(4, 1), (3, 1), (5, 4), (2, 2), (1, 4), (3, 2), (1, 1), (4, 2),
                                   (3, 3), (5, 1), (1, 5), (5, 5), (3, 4)])
@pytest.mark.parametrize("shape,rho_fixed", I8_SHAPES)
def test_slice_products_i8_bit_exact(ll, nh, nl, shape, rho_fixed):
    N, K, M = shape
    A, B = gen("randn", (N, K), 5), gen("wide2", (K, M), 6)
    a, b, (oa, oae, ob, obe), sched, rho = _slices_i8(ll, A, B, nh, nl, rho_fixed)
    case(f"ozk_slice_products_i8 ({nh},{nl}) N,K,M={shape} rho={rho}")
    P = to_np(ll.slice_products(a, b, ll.PIPE_ONDEVICE, nh, nl))
    unit = 2.0 ** (rho - 24)
    assert OP.products_exact_certificate(oa, ob, sched, unit, unit)
    assert np.array_equal(P, O.slice_products(oa, ob, sched))


@pytest.mark.parametrize("nh,nl", [(4, 1), (3, 1), (5, 4), (2, 2), (1, 4), (3, 2), (1, 1), (4, 2),
                                   (3, 3), (5, 1), (1, 5), (5, 5), (3, 4), (6, 1), (1, 6),
                                   (6, 5), (7, 6), (8, 8), (8, 3), (3, 8)])
@pytest.mark.parametrize("shape,rho_fixed", I8_SHAPES)
def test_gemm_i8_orders_bit_exact(ll, nh, nl, shape, rho_fixed):
    N, K, M = shape
    A, B = gen("wide2", (N, K), 7), gen("randn", (K, M), 8)
    a, b, (oa, oae, ob, obe), sched, rho = _slices_i8(ll, A, B, nh, nl, rho_fixed)
    Pref = O.slice_products(oa, ob, sched)
    case(f"ozk_gemm_i8 ({nh},{nl}) order A4 N,K,M={shape} rho={rho}")
    C = to_np(ll.gemm(a, b, ll.PIPE_ONDEVICE, nh, nl, ll.ORDER_2SUM))
    assert np.array_equal(C, OP.combine_f64(*O.accumulate_a4(Pref, sched, oae, obe)))
    case(f"ozk_gemm_i8 ({nh},{nl}) order A3 N,K,M={shape} rho={rho}")
    C = to_np(ll.gemm(a, b, ll.PIPE_ONDEVICE, nh, nl, ll.ORDER_BLOCK64))
    assert np.array_equal(C, O.accumulate_a3(Pref, sched, oae, obe))


# ---------------------------------------------------------------- orders

ORDERS = {"ondevice": [("A4", 0), ("A3", 1)], "host": [("A2", 2), ("A1", 3)]}


@pytest.mark.parametrize("pipe,nh,nl", SCHEDULES)
@pytest.mark.parametrize("shape", [(96, 70, 160), (130, 257, 67), (2, 5, 3)])
def test_gemm_orders_bit_exact(ll, pipe, nh, nl, shape):
    N, K, M = shape
    A, B = gen("wide2", (N, K), 3), gen("randn", (K, M), 4)
    a, b, (oa, oae, ob, obe), sched, code = _slices(ll, A, B, pipe, nh, nl)
    Pref = O.slice_products(oa, ob, sched)
    refs = {"A4": lambda: OP.combine_f64(*O.accumulate_a4(Pref, sched, oae, obe)),
            "A3": lambda: O.accumulate_a3(Pref, sched, oae, obe),
            "A2": lambda: O.accumulate_a2(Pref, sched, oae, obe),
            "A1": lambda: O.accumulate_a1(Pref, sched, oae, obe)}
    for name, code_o in ORDERS[pipe]:
        case(f"ozk_gemm {pipe} ({nh},{nl}) order {name} N,K,M={shape}")
        C = to_np(ll.gemm(a, b, code, nh, nl, code_o))
        assert np.array_equal(C, refs[name]()), name


# ---------------------------------------------------------------- public API

@pytest.mark.parametrize("precision", ["high", "medium", "max", (4, 2), (2, 2), (1, 1), (1, 2),
                                       (1, 4), (2, 1), (2, 3), (3, 2), (3, 3), (2, 4), (4, 4),
                                       (5, 1), (5, 2), (5, 3), (5, 5), (4, 3), (4, 5), (3, 4),
                                       (3, 5), (2, 5), (1, 5), (6, 1), (1, 6), (6, 5),
                                       (7, 6), (8, 8), (2, 7), (9, 1)])
@pytest.mark.parametrize("accumulation", ["fused", "bf16_interleaved", "ondevice", "host"])
def test_matmul_ondevice_bit_exact(ozk, precision, accumulation):
    A, B = gen("randn", (150, 300), 21), gen("randn", (300, 90), 22)
    case(f"matmul ondevice {precision} {accumulation} (150,300,90)")
    C = ozk.matmul(A, B, pipeline="ondevice", accumulation=accumulation,
                   precision=precision)
    nh, nl = OP.resolve_precision(precision)
    if accumulation == "host":
        ref = O.matmul_ondevice_a3(A, B, "raise", nh, nl)
    else:
        ref = O.matmul_ondevice_a4(A, B, "raise", nh, nl)
    assert isinstance(C, np.ndarray) and C.dtype == np.float64
    assert np.array_equal(C, ref)
    assert np.all(np.abs(C - ref) <= 2.0 ** -51 * (np.abs(A) @ np.abs(B)))


@pytest.mark.parametrize("precision", ["high", "medium", "max", (1, 1), (1, 2), (1, 3), (2, 1),
                                       (2, 2), (2, 3), (3, 2), (3, 3), (4, 2), (2, 4), (4, 4),
                                       (5, 1), (5, 2), (5, 3), (5, 5), (4, 3), (4, 5), (3, 4),
                                       (3, 5), (2, 5), (1, 5), (6, 1), (1, 6), (6, 5),
                                       (7, 6), (8, 8), (8, 2), (9, 1)])
def test_matmul_long_contraction_bit_exact(ozk, precision):
    # K > 4096: rho >= 19, every schedule with both counts in 1 .. 8 runs on
    # INT8 planes in the all-pairs kernel (one, two or three sweeps up to 5,
    # rectangle sweeps beyond); (9, 1) on BF16 planes in the pairwise kernel
    A, B = gen("randn", (40, 6000), 23), gen("wide2", (6000, 70), 24)
    nh, nl = OP.resolve_precision(precision)
    for acc, ref in [("fused", lambda: O.matmul_ondevice_a4(A, B, "raise", nh, nl)),
                     ("host", lambda: O.matmul_ondevice_a3(A, B, "raise", nh, nl))]:
        case(f"matmul ondevice {precision} {acc} (40,6000,70)")
        C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=precision)
        assert np.array_equal(C, ref())


@pytest.mark.parametrize("K", [5000, 8192, 4100])
@pytest.mark.parametrize("aligned", [True, False])
def test_matmul_operand_strides_bit_exact(ozk, K, aligned):
    """Torch views with odd leading dimensions and, unaligned, an 8-byte
    offset (element-wise loads for both operands), at K where A's rows fit
    one workgroup and B's columns are extracted in place by gangs.  N = 65
    and M = 70 leave padding lines in both plane sets."""
    import torch
    N, M = 65, 70
    rng = np.random.RandomState(K + aligned)
    Abig = torch.tensor(rng.randn(N, K + 3), device="cuda")
    Bbig = torch.tensor((rng.rand(K, M + 3) - 0.5) * np.exp(2.0 * rng.randn(K, M + 3)),
                        device="cuda")
    o = 0 if aligned else 1
    At, Bt = Abig[:, o:o + K], Bbig[:, o:o + M]
    A, B = At.cpu().numpy(), Bt.cpu().numpy()
    for precision in ("high", "medium", (5, 1), (6, 1)):
        nh, nl = OP.resolve_precision(precision)
        case(f"matmul strided views ({N},{K},{M}) aligned={aligned} {precision}")
        C = ozk.matmul(At, Bt, pipeline="ondevice", precision=precision)
        assert np.array_equal(C.cpu().numpy(), O.matmul_ondevice_a4(A, B, "raise", nh, nl))


def _tail_split(ntiles, K, i8, cus=256, min_piece=16):
    """Pieces per tail tile of the all-pairs kernel's K-split tail on a GPU
    with `cus` CUs (MI355X: 256): 0 when the product does not split."""
    nst = -(-K // 64) * 64 * (1 if i8 else 2) // 64
    T = ntiles % cus
    if T == 0:
        return 0
    P = min(cus // T, nst // min_piece)
    return P if P >= 2 else 0


# Products whose tile count leaves a partial last round: the tail tiles are
# split along K over the workgroups, their raw sums added by the fixup
# kernel, then folded.  (N, K, M): 100 tiles in no full round; 324 tiles =
# one round + 68 split tail tiles; BF16 planes (K <= 4096) with 121 tiles.
@pytest.mark.parametrize("N,K,M", [(640, 8192, 640), (1100, 8192, 1100), (700, 4096, 700)])
@pytest.mark.parametrize("precision", ["high", "medium"])
def test_matmul_tail_split_bit_exact(ozk, N, K, M, precision):
    ntiles = -(-N // 64) * -(-M // 64)
    assert _tail_split(ntiles, K, K > 4096) >= 2  # the case exercises the split
    A, B = gen("wide2", (N, K), N + 1), gen("randn", (K, M), M + 2)
    nh, nl = OP.resolve_precision(precision)
    rows = np.r_[0:40, N // 2:N // 2 + 24, N - 40:N]  # the last tile rows are tail tiles
    for acc in ("fused", "host"):
        case(f"matmul tail split {precision} {acc} ({N},{K},{M})")
        C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=precision)
        ref = (O.matmul_ondevice_a3(A[rows], B, "raise", nh, nl) if acc == "host"
               else O.matmul_ondevice_a4(A[rows], B, "raise", nh, nl))
        assert np.array_equal(C[rows], ref)


# Multi-sweep schedules on a partial last round (their sweeps do not split
# the tail along K; the fold state crosses sweeps): 1100 x 1100 gives 324
# tiles of 64 rows (one round and 68 tiles on 256 CUs) and 216 of 96 rows.
# max (three sweeps), (4, 2) (two), (6, 1) and (7, 6) (rectangle sweeps);
# INT8 planes (K = 6000) and BF16 (K = 3000); orders A4 and A3.
@pytest.mark.parametrize("precision", ["max", (4, 2), (6, 1), (7, 6)])
@pytest.mark.parametrize("K", [6000, 3000])
def test_matmul_multisweep_partial_round_bit_exact(ozk, precision, K):
    N = M = 1100
    A, B = gen("wide2", (N, K), 91), gen("randn", (K, M), 92)
    nh, nl = OP.resolve_precision(precision)
    rows = np.r_[0:8, N // 2:N // 2 + 8, N - 16:N]
    for acc in ("fused", "host"):
        case(f"matmul multi-sweep partial round {precision} {acc} ({N},{K},{M})")
        C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=precision)
        ref = (O.matmul_ondevice_a3(A[rows], B, "raise", nh, nl) if acc == "host"
               else O.matmul_ondevice_a4(A[rows], B, "raise", nh, nl))
        assert np.array_equal(C[rows], ref)


def test_host_multisweep_partial_round_bit_exact(ozk):
    """The host triangle of 8 slices in its three sweeps on a partial last
    round: 1100 x 1100 (324 tiles of 64 rows), K = 1024 on BF16 planes.  A2
    through matmul, A1 through matmul_numpy."""
    N, K, M = 1100, 1024, 1100
    A, B = gen("wide2", (N, K), 93), gen("randn", (K, M), 94)
    rows = np.r_[0:16, 540:556, N - 24:N]
    case(f"matmul host 8 slices {(N, K, M)} (multi-sweep, partial round)")
    C = ozk.matmul(A, B, n_slices=8)
    assert np.array_equal(C[rows], OP.matmul_host_a2(A[rows], B, n_slices=8))
    C = ozk.matmul_numpy(A, B, n_slices=8)
    assert np.array_equal(C[rows], O.matmul_numpy(A[rows], B, n_slices=8))


def test_host_schedule_tail_split_bit_exact(ll):
    """The host triangle of 5 slices runs in one all-pairs sweep, which
    splits its tail along K when the workspace has room for the partial
    sums: 17 x 17 = 289 tiles leave 33 tail tiles, each in 2 pieces of 16
    stages (K = 1024 on BF16 planes).  Orders A2 and A1 against the oracle
    on the tail rows and others, split and in the static order (the
    workspace ozk_gemm_workspace_bytes gives, which has no K)."""
    N, K, M = 1088, 1024, 1088
    assert _tail_split(17 * 17, K, False) == 2
    A, B = gen("wide2", (N, K), 41), gen("randn", (K, M), 42)
    a, b, (oa, oae, ob, obe), sched, code = _slices(ll, A, B, "host", 5, 0)
    rows = np.r_[0:16, 500:520, N - 48:N]
    Pref = O.slice_products(oa[:, rows], ob, sched)
    for name, code_o, acc in (("A2", 2, O.accumulate_a2), ("A1", 3, O.accumulate_a1)):
        for ws, how in ((64 << 20, "K-split tail"), (None, "static order")):
            case(f"ozk_gemm host 5 slices order {name} N,K,M={(N, K, M)} ({how})")
            C = to_np(ll.gemm(a, b, code, 5, 0, code_o, workspace_bytes=ws))
            assert np.array_equal(C[rows], acc(Pref, sched, oae[:, rows], obe)), name


@pytest.mark.parametrize("precision", ["high", "medium"])
def test_gram_tail_split_bit_exact(ozk, precision):
    # 640 columns: 55 upper tiles of K = 8192 stages split 4 ways each
    A = gen("randn", (8192, 640), 71)
    assert _tail_split(10 * 11 // 2, 8192, True) == 4
    case(f"gram tail split {precision} (8192,640)")
    G = ozk.gram(A, mode="ozaki", precision=precision)
    assert np.array_equal(G, O.gram_ozaki(A, precision))
    assert np.array_equal(G, G.T)


def test_matmul_numpy_bit_exact(ozk):
    A, B = gen("wide2", (70, 200), 31), gen("wide2", (200, 50), 32)
    case("matmul_numpy host / ondevice (70,200,50)")
    assert np.array_equal(ozk.matmul_numpy(A, B), O.matmul_numpy(A, B))
    assert np.array_equal(ozk.matmul_numpy(A, B, pipeline="ondevice"),
                          O.matmul_numpy(A, B, pipeline="ondevice"))
    assert np.array_equal(ozk.matmul_numpy(A, B, pipeline="ondevice", precision="max"),
                          O.matmul_numpy(A, B, pipeline="ondevice", precision="max"))
    case("matmul host (70,200,50)")
    assert np.array_equal(ozk.matmul(A, B), OP.matmul_host_a2(A, B))
    assert np.array_equal(ozk.matmul(A, B, n_slices=9), OP.matmul_host_a2(A, B, n_slices=9))


def test_matmul_host_nine_slices_k4096_bit_exact(ozk):
    """K = 4096: rho = 47 leaves 6 bits per slice, so the host pipeline's
    safety budget (matmul.py:102-106) needs 9 slices; they run in the
    all-pairs kernel's four sweeps (45 pairs).  Rows across the 64-row
    tiles, A2 and A1."""
    A, B = gen("randn", (200, 4096), 35), gen("wide2", (4096, 150), 36)
    rows = np.r_[0:3, 63:66, 197:200]
    case("matmul host (200,4096,150) n_slices=9")
    C = ozk.matmul(A, B, n_slices=9)
    assert np.array_equal(C[rows], OP.matmul_host_a2(A[rows], B, n_slices=9))
    C = ozk.matmul_numpy(A, B, n_slices=9)
    assert np.array_equal(C[rows], O.matmul_numpy(A[rows], B, n_slices=9))


@pytest.mark.parametrize("n_slices", [8, 9, 10])
def test_matmul_host_tiles_bit_exact(ozk, n_slices):
    """The host pipeline on several tiles with partial edges: 8 slices run
    the all-pairs kernel's three sweeps, 9 its four, 10 the pairwise kernel;
    A2 through matmul, A1 through matmul_numpy."""
    A, B = gen("wide2", (300, 1000), 33), gen("wide2", (1000, 260), 34)
    case(f"matmul host (300,1000,260) n_slices={n_slices}")
    assert np.array_equal(ozk.matmul(A, B, n_slices=n_slices),
                          OP.matmul_host_a2(A, B, n_slices=n_slices))
    assert np.array_equal(ozk.matmul_numpy(A, B, n_slices=n_slices),
                          O.matmul_numpy(A, B, n_slices=n_slices))


def _digest(a):
    import hashlib
    a = np.ascontiguousarray(a)
    return hashlib.sha256(a.tobytes()).hexdigest() + f":{a.dtype}:{a.shape}"


def test_config1_host_256(ozk, ll, golden_dir):
    """256x256 RandomState(0), n_slices=8, host pipeline: slices, exponents,
    each per-pair product and C bit-exact against the committed digests."""
    doc = json.loads((golden_dir / "config1.json").read_text())
    rs = np.random.RandomState(0)
    A, B = rs.randn(256, 256), rs.randn(256, 256)
    case("config1 host 256: extraction + products + matmul_numpy")
    a = ll.extract(A, 0, doc["rho64"], 8, f64=True)
    b = ll.extract(B, 1, doc["rho64"], 8, f64=True)
    assert _digest(to_np(a.values())) == doc["a_slices"]
    assert _digest(to_np(a.exponents())) == doc["a_exps"]
    assert _digest(to_np(b.values()).transpose(0, 2, 1)) == doc["b_slices_cols"]
    assert _digest(to_np(b.exponents())) == doc["b_exps"]
    assert _digest(to_np(ll.slice_products(a, b, ll.PIPE_HOST, 8, 0))) == doc["products"]
    C = ozk.matmul_numpy(A, B)
    assert _digest(C) == doc["C_numpy_order"]
    assert _digest(ozk.matmul(A, B)) == doc["C_jax_order"]


def _exact(A, B):
    from fractions import Fraction
    Af = [[Fraction(float(v)) for v in r] for r in A]
    Bf = [[Fraction(float(v)) for v in r] for r in B]
    return np.array([[float(sum(Af[i][t] * Bf[t][j] for t in range(A.shape[1])))
                      for j in range(B.shape[1])] for i in range(A.shape[0])])


def test_error_vs_exact_no_worse_than_reference(ozk):
    A, B = gen("wide2", (7, 48), 41), gen("wide2", (48, 6), 42)
    ex = _exact(A, B)
    case("exact-rational comparison (7,48,6)")
    for kw, ref in [({"pipeline": "ondevice"}, O.matmul_ondevice_a4(A, B)),
                    ({"pipeline": "ondevice", "precision": "max"},
                     O.matmul_ondevice_a4(A, B, "raise", 5, 4)),
                    ({}, OP.matmul_host_a2(A, B))]:
        C = ozk.matmul(A, B, **kw)
        assert np.all(np.abs(C - ex) <= np.abs(ref - ex)), kw


def test_ragged_and_degenerate_shapes(ozk):
    for N, K, M in [(1, 1, 1), (1, 700, 1), (65, 1, 63), (3, 64, 200), (0, 5, 4), (4, 5, 0)]:
        A, B = gen("randn", (N, K), N + K), gen("randn", (K, M), K + M)
        case(f"matmul ondevice ragged {N},{K},{M}")
        C = ozk.matmul(A, B, pipeline="ondevice")
        assert C.shape == (N, M)
        if N and M:
            assert np.array_equal(C, O.matmul_ondevice_a4(A, B))
    with pytest.raises(ValueError):
        ozk.matmul(np.ones((2, 0)), np.ones((0, 2)), pipeline="ondevice")


def test_preflight_and_families(ozk):
    import torch
    A = gen("randn", (8, 16), 1)
    B = gen("randn", (16, 4), 2)
    case("preflight errors")
    bad = A.copy()
    bad[1, 1] = np.nan
    with pytest.raises(ValueError, match="NaN or Inf"):
        ozk.matmul(bad, B, pipeline="ondevice")
    fb = ozk.matmul(bad, B, pipeline="ondevice", safe_mode="fallback")
    assert np.isnan(fb[1]).all() and np.allclose(fb[0], (bad @ B)[0], rtol=1e-14)
    with pytest.raises(ValueError, match="Unknown accumulation"):
        ozk.matmul(A, B, pipeline="ondevice", accumulation="x")
    with pytest.raises(ValueError, match="Unknown precision"):
        ozk.matmul(A, B, pipeline="ondevice", precision="x")
    with pytest.raises(ValueError, match="Unknown pipeline"):
        ozk.matmul(A, B, pipeline="x")
    with pytest.raises(ValueError, match="Invalid safe_mode"):
        ozk.matmul(A, B, pipeline="ondevice", safe_mode="x")
    with pytest.raises(ValueError, match="both be numpy"):
        ozk.matmul(torch.tensor(A), B, pipeline="ondevice")
    case("safe_mode fallback (2,10000)@(10000,2)")
    rng = np.random.RandomState(0)
    Ab, Bb = rng.randn(2, 10000), rng.randn(10000, 2)
    with pytest.raises(ValueError, match="insufficient slice budget"):
        ozk.matmul(Ab, Bb)
    Cf = ozk.matmul(Ab, Bb, safe_mode="fallback")
    assert rel_err(Cf, Ab @ Bb) <= 1e-14
    case("torch family on device")
    At = torch.tensor(A, device="cuda")
    Bt = torch.tensor(B, device="cuda")
    Ct = ozk.matmul(At, Bt, pipeline="ondevice")
    assert isinstance(Ct, torch.Tensor) and Ct.is_cuda
    assert np.array_equal(Ct.cpu().numpy(), O.matmul_ondevice_a4(A, B))
    Ch = ozk.matmul(At, Bt)   # host pipeline always returns NumPy
    assert isinstance(Ch, np.ndarray)
    # non-contiguous views are accepted
    Av = torch.tensor(gen("randn", (16, 8), 3), device="cuda").T
    Cv = ozk.matmul(Av, Bt, pipeline="ondevice")
    assert np.array_equal(Cv.cpu().numpy(), O.matmul_ondevice_a4(Av.cpu().numpy(), B))


# ---------------------------------------------------------------- gram / residual / solve

# (4500, 600): 10 x 10 tiles of 64 (two tile-row groups of the upper-triangle
# order, a ragged last tile), INT8 planes; max takes the full product and a
# separate symmetrisation, and so do the custom schedules: (4, 2) in two
# fixed sweeps, (6, 1) and (7, 6) in rectangle sweeps over one plane set.
@pytest.mark.parametrize("shape", [(64, 64), (300, 40), (33, 130), (5000, 24), (4500, 600)])
@pytest.mark.parametrize("precision", ["high", "medium", "max", (4, 2), (6, 1), (7, 6)])
def test_gram_bit_exact(ozk, shape, precision):
    A = gen("randn", shape, 51)
    case(f"gram ozaki {shape} {precision}")
    for acc in ("bf16_interleaved", "fused"):
        G = ozk.gram(A, mode="ozaki", precision=precision, accumulation=acc)
        assert np.array_equal(G, O.gram_ozaki(A, precision))
        assert np.array_equal(G, G.T)


@pytest.mark.parametrize("shape", [(64, 64), (200, 50), (37, 300), (20, 5000)])
def test_residual_bit_exact(ozk, shape):
    N, K = shape
    rng = np.random.RandomState(61)
    A, x, b = rng.randn(N, K), rng.randn(K), rng.randn(N)
    case(f"residual ozaki {shape}")
    r = ozk.residual(A, x, b, mode="ozaki")
    assert r.shape == (N,) and np.array_equal(r, O.residual_ozaki(A, x, b))
    X, Bm = rng.randn(K, 3), rng.randn(N, 3)
    R = ozk.residual(A, X, Bm, mode="ozaki", accumulation="fused")
    assert np.array_equal(R, O.residual_ozaki(A, X, Bm))


@pytest.mark.parametrize("N,K", [(37, 1), (37, 1100), (129, 4096), (5, 513), (70, 2049),
                                 (33, 3000), (40, 8192), (300, 8192), (11, 5001), (9, 12000),
                                 (7, 9999), (17, 16384), (6, 16385)])
@pytest.mark.parametrize("precision", ["high", "medium", "max"])
def test_residual_fused_rows_bit_exact(ozk, N, K, precision):
    # high / medium: K <= 2048 runs the one-wave-per-row kernel, K <= 16384
    # the split-row kernel (4 waves of 1024 elements up to K = 4096, then 8
    # waves of 1024 or 2048, their rows through an LDS ring when K is even,
    # else the register prefetch: 5001, 9999); K = 16385 takes the
    # slice-GEMM route.  max: one wave per row up to K = 1024, then 2, 4 or
    # 8 waves of 1024 elements up to K = 8192 (5001 without the ring), the
    # slice-GEMM route beyond
    rng = np.random.RandomState(N + K)
    A = (rng.rand(N, K) - 0.5) * np.exp(2.0 * rng.randn(N, K))
    x, b = rng.randn(K), rng.randn(N)
    case(f"residual fused rows {precision} N={N} K={K}")
    r = ozk.residual(A, x, b, mode="ozaki", precision=precision)
    assert np.array_equal(r, O.residual_ozaki(A, x, b, precision))


@pytest.mark.parametrize("K,ncols", [(700, 2), (2048, 4), (5000, 3), (9000, 5)])
def test_residual_fused_columns_bit_exact(ozk, K, ncols):
    # up to 4 right-hand sides run the row kernels once per column; 5 take
    # the slice-GEMM route; x and b strided (columns of matrices)
    rng = np.random.RandomState(K + ncols)
    N = 150
    A = rng.randn(N, K) * np.exp(rng.randn(N, 1))
    X, Bm = rng.randn(K, ncols), rng.randn(N, ncols)
    case(f"residual fused columns K={K} ncols={ncols}")
    R = ozk.residual(A, X, Bm, mode="ozaki")
    assert R.shape == (N, ncols)
    assert np.array_equal(R, O.residual_ozaki(A, X, Bm))


@pytest.mark.parametrize("K", [2048, 1500, 1024, 700, 4096, 6000, 16384])
@pytest.mark.parametrize("precision", ["high", "medium", "max"])
def test_residual_rows_batches_and_edge_rows(ozk, K, precision):
    """40000 rows (fewer for K > 2048, about 80 M elements): every wave of
    the one-wave-per-row kernel's persistent grid (one workgroup of 8 waves
    per CU), and every workgroup of the split-row kernel's, takes more than
    one batch of 16 rows, the last one partial.  K = 2048 / 1024 / 4096 /
    16384 are whole rows of the kernels, 1500 / 700 / 6000 take the guarded
    loads.  Special rows: all zero (no slice), one nonzero,
    scaled by 2^-103 (slice exponents below -100: normalised dot products,
    subnormal lo parts), 2^105 (exponents above 100), a wide row, and one
    scaled by 2^-110, where 2^-c overflows FP32 in the reference's
    extraction and its result is NaN (extract.py:145-148; at K = 1024 the
    2^-103 row's last slices do too); the kernel must give NaN there too.  Rows are independent, so three row ranges are
    checked against the oracle on those rows alone."""
    N = 40000 if K <= 2048 else 80_000_000 // K
    rng = np.random.RandomState(K + {"high": 7, "medium": 11, "max": 13}[precision])
    A = rng.randn(N, K)
    A[3] = 0.0
    A[5] = 0.0
    A[5, 7] = 1.5
    A[100] *= 2.0 ** -103
    A[101] *= 2.0 ** 105
    A[102] = rng.randn(K) * np.exp(3.0 * rng.randn(K))
    A[N - 2] *= 2.0 ** -110
    x, b = rng.randn(K), rng.randn(N)
    b[[3, 5, 100, 101, 102, N - 2]] = 0.0  # r = -Ozaki(A, x) exactly there
    case(f"residual rows N={N} K={K} {precision}")
    r = ozk.residual(A, x, b, mode="ozaki", precision=precision)
    sel = np.r_[0:300, N // 2:N // 2 + 100, N - 300:N]
    with np.errstate(over="ignore", invalid="ignore"):
        ref = O.residual_ozaki(A[sel], x, b[sel], precision)
    assert np.isnan(ref[-2]) and np.isfinite(ref).sum() >= len(sel) - 2
    assert np.array_equal(r[sel], ref, equal_nan=True)


@pytest.mark.parametrize("K", [2048, 700, 4096, 9000, 20000])
def test_residual_flags_through_c_abi(ozk, K):
    """ozk_residual clears the flag word itself, whatever it held, and sets
    OZK_FLAG_NONFINITE for a NaN/Inf in x or in A: on the fused row paths
    (K <= 16384), where the row kernels write the word, and on the
    slice-GEMM path (K = 20000)."""
    import torch
    from ozaki_jax_amd import _lib, _device as D
    lib = _lib.load()
    dev = torch.device("cuda", 0)
    rng = np.random.RandomState(K)
    N = 300
    A = torch.from_numpy(rng.randn(N, K)).to(dev)
    x = torch.from_numpy(rng.randn(K, 1)).to(dev)
    b = torch.from_numpy(rng.randn(N, 1)).to(dev)
    r = torch.empty((N, 1), dtype=torch.float64, device=dev)
    wsb = lib.ozk_residual_workspace_bytes(N, K, 1, 4, 1)
    ws = D.workspace(wsb, dev)

    def run(A_, x_):
        flags = torch.full((1,), -559038737, dtype=torch.int32, device=dev)
        _lib.check(lib.ozk_residual(
            A_.data_ptr(), D.ld_of(A_), x_.data_ptr(), D.ld_of(x_), b.data_ptr(),
            D.ld_of(b), r.data_ptr(), D.ld_of(r), N, K, 1, 4, 1, ws.data_ptr(),
            wsb, flags.data_ptr(), D.stream_handle()))
        return int(flags.item()) & 0xffffffff

    case(f"residual flags K={K}")
    assert run(A, x) == 0
    x2 = x.clone()
    x2[K // 3, 0] = float("nan")
    assert run(A, x2) == _lib.OZK_FLAG_NONFINITE
    A2 = A.clone()
    A2[N - 1, K - 1] = float("inf")
    assert run(A2, x) == _lib.OZK_FLAG_NONFINITE


def test_known_answers_on_gpu(ozk, golden_dir):
    """gram / residual errors recorded by the reference (tpu_full_results.json
    :77,93,109,157,173,189) from the same RandomState(42) draws."""
    known = json.loads((golden_dir / "reference_known_answers.json").read_text())["tpu_full_results"]
    rng = np.random.RandomState(42)
    for n in [64, 128, 256]:
        rng.randn(n, n), rng.randn(n, n)
    rng.randn(128, 128), rng.randn(128, 128), rng.randn(64, 256), rng.randn(256, 32)
    for n in [64, 128, 256]:
        A = rng.randn(n, n)
        case(f"known answer gram n={n}")
        e = rel_err(ozk.gram(A, mode="ozaki"), A.T @ A)
        assert e == pytest.approx(known[f"gram ozaki n={n}"]["error"], rel=1e-6)
    rng.randn(256, 64), rng.randn(128, 128)
    for n in [64, 128, 256]:
        A, x, b = rng.randn(n, n), rng.randn(n), rng.randn(n)
        case(f"known answer residual n={n}")
        e = rel_err(ozk.residual(A, x, b, mode="ozaki"), b - A @ x)
        assert e == pytest.approx(known[f"residual ozaki n={n}"]["error"], rel=1e-6)


def test_solve_ozaki(ozk):
    """ci_solve_validate.py:49-71 thresholds; FP32 LU comes from a different
    LAPACK than the oracle's, so the comparison is by tolerance."""
    rng = np.random.RandomState(42)
    n = 128
    A, b = rng.randn(n, n), rng.randn(n)
    xr = np.linalg.solve(A, b)
    case("solve ozaki n=128")
    assert rel_err(ozk.solve(A, b, residual_mode="ozaki"), xr) <= 1e-7
    assert rel_err(ozk.solve(A, b, residual_mode="ozaki", precision="medium"), xr) <= 1e-5
    assert rel_err(ozk.solve(A, b, residual_mode="ozaki", accumulation="fused"), xr) <= 1e-7
    assert rel_err(ozk.solve(A, b), xr) <= 1e-12
    e0 = rel_err(ozk.solve(A, b, max_iterations=0), xr)
    e1 = rel_err(ozk.solve(A, b, max_iterations=1), xr)
    e3 = rel_err(ozk.solve(A, b, max_iterations=3), xr)
    assert e1 < e0 * 1e-4 and e3 < e1
    X = ozk.solve(A, rng.randn(n, 4), residual_mode="ozaki")
    assert X.shape == (n, 4)
    with pytest.raises(ValueError, match="square"):
        ozk.solve(rng.randn(3, 4), rng.randn(3))


def test_extract_api_helpers(ozk):
    X = gen("wide2", (20, 33), 71)
    case("extract_split_* API helpers")
    s, e = ozk.extract_split_rows(X, O.rho_f64(33), 8)
    rs, re_ = O.extract_rows_f64(X, O.rho_f64(33), 8)
    assert np.array_equal(np.stack(s), rs) and np.array_equal(np.stack(e), re_)
    s, e = ozk.f32_extract_split_cols(X.astype(np.float32), O.rho_f32(20), 5)
    rs, re_ = O.extract_cols_f32(X.astype(np.float32), O.rho_f32(20), 5)
    assert np.array_equal(np.stack(s), rs) and np.array_equal(np.stack(e), re_)
    st, et = ozk.jax_extract_split_rows(X.astype(np.float32), 17, 4)
    rs, re_ = O.extract_rows_f32(X.astype(np.float32), 17, 4)
    assert np.array_equal(st, rs) and np.array_equal(et, re_)
