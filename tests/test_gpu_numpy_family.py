"""The NumPy family runs without PyTorch.

The reference's matmul_numpy and the NumPy branch of matmul need nothing but
NumPy (matmul.py:823-858).  Here NumPy inputs go through the HIP runtime and
rocBLAS by ctypes (ozaki_jax_amd._hip); PyTorch is only the optional tensor
family.  These tests replace the package's torch module with a stub that
fails on any use, then run matmul / matmul_numpy / gram / residual on NumPy
inputs against the oracle, bit for bit.
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


class _NoTorch:
    def __getattr__(self, name):
        raise AssertionError(f"torch.{name} used by the NumPy family")


@pytest.fixture
def no_torch(ozk, monkeypatch):
    from ozaki_jax_amd import _device as D
    monkeypatch.setattr(D, "torch", _NoTorch())
    return ozk


def test_matmul_without_torch(no_torch):
    ozk = no_torch
    rng = np.random.RandomState(3)
    for (N, K, M), prec, acc in [((150, 300, 90), "high", "fused"),
                                 ((150, 300, 90), "max", "host"),
                                 ((40, 6000, 70), "high", "fused"),
                                 ((40, 6000, 70), "medium", "host")]:
        A, B = rng.randn(N, K), rng.randn(K, M)
        nh, nl = OP.resolve_precision(prec)
        case(f"matmul ondevice {prec} {acc} ({N},{K},{M}) without torch")
        C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=prec)
        f = O.matmul_ondevice_a3 if acc == "host" else O.matmul_ondevice_a4
        assert isinstance(C, np.ndarray) and np.array_equal(C, f(A, B, "raise", nh, nl))
    A, B = rng.randn(70, 200), rng.randn(200, 50)
    case("matmul host pipeline without torch")
    assert np.array_equal(ozk.matmul(A, B), OP.matmul_host_a2(A, B))
    case("matmul_numpy host / ondevice without torch (lists accepted)")
    assert np.array_equal(ozk.matmul_numpy(A.tolist(), B.tolist()), O.matmul_numpy(A, B))
    assert np.array_equal(ozk.matmul_numpy(A, B, pipeline="ondevice", precision="max"),
                          O.matmul_numpy(A, B, pipeline="ondevice", precision="max"))


def test_preflight_and_fallback_without_torch(no_torch):
    ozk = no_torch
    rng = np.random.RandomState(4)
    A, B = rng.randn(8, 16), rng.randn(16, 4)
    bad = A.copy()
    bad[1, 1] = np.nan
    case("preflight NaN without torch")
    with pytest.raises(ValueError, match="NaN or Inf"):
        ozk.matmul(bad, B, pipeline="ondevice")
    case("safe_mode fallback (rocBLAS DGEMM) without torch")
    fb = ozk.matmul(bad, B, pipeline="ondevice", safe_mode="fallback")
    assert np.isnan(fb[1]).all() and np.allclose(fb[0], (bad @ B)[0], rtol=1e-14)
    Ab, Bb = rng.randn(2, 10000), rng.randn(10000, 2)
    Cf = ozk.matmul(Ab, Bb, safe_mode="fallback")  # host pipeline: unsafe budget
    assert np.allclose(Cf, Ab @ Bb, rtol=1e-13, atol=1e-12)


def test_gram_and_residual_without_torch(no_torch):
    ozk = no_torch
    rng = np.random.RandomState(5)
    for shape, prec in [((300, 40), "high"), ((5000, 24), "max"), ((8192, 70), "high")]:
        A = rng.randn(*shape)
        case(f"gram ozaki {shape} {prec} without torch")
        G = ozk.gram(A, mode="ozaki", precision=prec)
        assert np.array_equal(G, O.gram_ozaki(A, prec)) and np.array_equal(G, G.T)
    A = rng.randn(200, 64)
    case("gram f64 (rocBLAS) without torch")
    G = ozk.gram(A)
    assert np.array_equal(G, G.T) and np.allclose(G, A.T @ A, rtol=1e-13, atol=1e-12)
    for (N, K), nc in [((300, 2048), None), ((37, 5000), None), ((64, 700), 3)]:
        A = rng.randn(N, K)
        x = rng.randn(K) if nc is None else rng.randn(K, nc)
        b = rng.randn(N) if nc is None else rng.randn(N, nc)
        case(f"residual ozaki ({N},{K}) ncols={nc} without torch")
        r = ozk.residual(A, x, b, mode="ozaki")
        assert r.shape == b.shape
        assert np.array_equal(r, O.residual_ozaki(A, x, b))
        case(f"residual f64 (rocBLAS) ({N},{K}) without torch")
        r = ozk.residual(A, x, b)
        assert np.allclose(r, b - A @ x, rtol=1e-12, atol=1e-10)
    A = rng.randn(40, 8192)
    A[3] *= 2.0 ** 110
    x, b = rng.randn(8192), rng.randn(40)
    case("residual ozaki with an overflowing row, without torch")
    with warnings.catch_warnings(), np.errstate(all="ignore"):
        warnings.simplefilter("ignore")
        ref = O.residual_ozaki(A, x, b)
    assert np.array_equal(ozk.residual(A, x, b, mode="ozaki"), ref, equal_nan=True)


def test_device_pool_reuses_blocks(no_torch):
    """Repeated calls of one shape take their device memory from the pool."""
    from ozaki_jax_amd import _hip
    ozk = no_torch
    A, B = np.random.RandomState(6).randn(256, 512), np.random.RandomState(7).randn(512, 128)
    ozk.matmul(A, B, pipeline="ondevice")
    pool = _hip._pool()
    before = sum(len(v) for v in pool.free.values())
    case("matmul x 3 on one shape: no new device blocks")
    calls = {"n": 0}
    real = pool.rt.malloc

    def counting(n):
        calls["n"] += 1
        return real(n)

    pool.rt.malloc = counting
    try:
        for _ in range(3):
            ozk.matmul(A, B, pipeline="ondevice")
    finally:
        pool.rt.malloc = real
    assert calls["n"] == 0 and sum(len(v) for v in pool.free.values()) >= before


@pytest.mark.parametrize("nbytes,chunk", [(5 * (1 << 20) + 24, 1 << 20), (2 << 20, 1 << 20),
                                          (3 << 20, 1 << 20), (1 << 20, 1 << 20),
                                          (4096 + 8, 1 << 20)])
def test_staged_transfers_round_trip(no_torch, nbytes, chunk):
    """Host copies through the pinned staging buffers: chunk boundaries,
    a final partial chunk, one and two chunks."""
    from ozaki_jax_amd import _hip
    rng = np.random.RandomState(nbytes % 1000)
    a = rng.randn(nbytes // 8)
    st = _hip._Stager(_hip._rt(), chunk)
    case(f"staged H2D / D2H of {a.nbytes} bytes in {chunk}-byte chunks")
    d = _hip.DeviceArray(a.shape)
    st.to_device(d.data_ptr(), a)
    assert np.array_equal(d.numpy(), a), "H2D"
    out = np.empty_like(a)
    st.to_host(out, d.data_ptr())
    assert np.array_equal(out, a), "D2H"


def test_large_array_round_trip(no_torch):
    """An array above the staging threshold goes through the default stager
    both ways."""
    from ozaki_jax_amd import _hip
    rng = np.random.RandomState(11)
    n = (_hip._STAGE_MIN + 2 * _hip._STAGE_CHUNK) // 8 + 1000
    a = rng.randn(n // 1000, 1000)
    case(f"DeviceArray round trip of {a.nbytes} bytes (staged)")
    d = _hip.DeviceArray.from_numpy(a)
    assert np.array_equal(d.numpy(), a)


def test_torch_staged_conversions(ozk):
    """NumPy <-> torch device conversions above the staging threshold (the
    torch family's inputs from NumPy and its NumPy outputs)."""
    import torch
    from ozaki_jax_amd import _device as D, _hip
    rng = np.random.RandomState(12)
    a = rng.randn(_hip._STAGE_MIN // 8 // 1000 + 700, 1000)
    dev = torch.device("cuda", torch.cuda.current_device())
    case(f"numpy -> torch -> numpy of {a.nbytes} bytes (staged)")
    t = D._numpy_to_torch(a, dev)
    assert t.device == dev and np.array_equal(t.cpu().numpy(), a)
    assert np.array_equal(D._torch_to_numpy(t * 2.0), a * 2.0)
    case("solve on NumPy input through the staged conversions")
    n = 2100
    A = rng.randn(n, n) + n * np.eye(n)
    b = rng.randn(n)
    x = ozk.solve(A, b)
    assert isinstance(x, np.ndarray) and np.linalg.norm(A @ x - b) <= 1e-12 * np.linalg.norm(b) * n


@pytest.mark.parametrize("shape,prec,acc,kind", [((2048, 4096, 4096), "high", "fused", None),
                                                 ((1100, 8192, 8192), "high", "fused", None),
                                                 ((1100, 8192, 8192), "medium", "host", "big"),
                                                 ((1100, 8192, 8192), "high", "fused", "nan")])
def test_numpy_matmul_in_row_halves(no_torch, monkeypatch, shape, prec, acc, kind):
    """Large NumPy products run as two calls on A's row halves, overlapping
    the transfers with the kernels: the same bits as the one-call path, and
    the same errors, fallbacks and reruns."""
    ozk = no_torch
    import importlib
    MM = importlib.import_module("ozaki_jax_amd.matmul")
    N, K, M = shape
    rng = np.random.RandomState(N + K)
    A, B = rng.randn(N, K), rng.randn(K, M)
    if kind == "big":
        A[7] *= 2.0 ** 110  # INF_SLICE in the FP64 block order: rerun on BF16 planes
    if kind == "nan":
        A[N - 3, 5] = np.nan
    assert MM._numpy_halves_ok(A, B)
    case(f"numpy matmul ondevice {prec} {acc} {shape} {kind}: halves vs one call")
    if kind == "nan":
        with pytest.raises(ValueError, match="NaN or Inf"):
            ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=prec)
        C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=prec,
                       safe_mode="fallback")
        monkeypatch.setattr(MM, "_numpy_halves_ok", lambda *a: False)
        C1 = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=prec,
                        safe_mode="fallback")
        assert np.array_equal(C, C1, equal_nan=True)
        return
    C = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=prec)
    Cn = ozk.matmul_numpy(A, B, pipeline="ondevice", precision=prec) if acc == "host" else None
    monkeypatch.setattr(MM, "_numpy_halves_ok", lambda *a: False)
    C1 = ozk.matmul(A, B, pipeline="ondevice", accumulation=acc, precision=prec)
    assert isinstance(C, np.ndarray) and np.array_equal(C, C1, equal_nan=True)
    if Cn is not None:
        assert np.array_equal(Cn, ozk.matmul_numpy(A, B, pipeline="ondevice", precision=prec),
                              equal_nan=True)
    rows = [0, 1, 575, 576, N - 1]
    nh, nl = OP.resolve_precision(prec)
    f = O.matmul_ondevice_a3 if acc == "host" else O.matmul_ondevice_a4
    case("sampled rows against the oracle")
    assert np.array_equal(C[rows[:4] if N > 576 else rows[:2]],
                          f(A[rows[:4] if N > 576 else rows[:2]], B, "raise", nh, nl),
                          equal_nan=True)


def test_extract_helpers_without_torch(no_torch):
    """extract_split_*, f32_extract_split_* and jax_extract_split_* on NumPy
    input (extract.py:21-286) with the planes unpacked on the host, bit for
    bit against the oracle; shapes cover the row kernels, the column gangs
    (8192 and 9000 rows) and the FP64 path's transposed columns."""
    ozk = no_torch
    rng = np.random.RandomState(21)
    for shape in [(20, 33), (96, 5000), (8192, 40), (9000, 24)]:
        X = (rng.rand(*shape) - 0.5) * np.exp(2.0 * rng.randn(*shape))
        X32 = X.astype(np.float32)
        r64, c64 = O.rho_f64(shape[1]), O.rho_f64(shape[0])
        r32, c32 = O.rho_f32(shape[1]), O.rho_f32(shape[0])
        case(f"extract helpers {shape} without torch")
        for got, ref in [
                (ozk.extract_split_rows(X, r64, 8), O.extract_rows_f64(X, r64, 8)),
                (ozk.extract_split_cols(X, c64, 8), O.extract_cols_f64(X, c64, 8)),
                (ozk.f32_extract_split_rows(X32, r32, 5), O.extract_rows_f32(X32, r32, 5)),
                (ozk.f32_extract_split_cols(X32, c32, 5), O.extract_cols_f32(X32, c32, 5))]:
            s, e = got
            assert isinstance(s[0], np.ndarray) and s[0].dtype == np.float32
            assert np.array_equal(np.stack(s), ref[0]) and np.array_equal(np.stack(e), ref[1])
            assert np.stack(e).dtype == ref[1].dtype
        st, et = ozk.jax_extract_split_rows(X32, r32, 4)
        rs, re_ = O.extract_rows_f32(X32, r32, 4)
        assert np.array_equal(st, rs) and np.array_equal(et, re_) and et.dtype == np.float32
        st, et = ozk.jax_extract_split_cols(X32, c32, 4)
        rs, re_ = O.extract_cols_f32(X32, c32, 4)
        assert np.array_equal(st, rs) and np.array_equal(et, re_)


def test_solve_inv_norm_without_torch(no_torch):
    """solve (FP32 LU and triangular solves of the library, FP64 or Ozaki
    residuals), inv and norm on NumPy input.  solve at n = 1024, cond 1e6,
    is within 2x of the oracle's refinement (NumPy's FP32 LAPACK solve, the
    oracle's Ozaki residuals) and 10x below the unrefined FP32 solve."""
    ozk = no_torch
    rng = np.random.RandomState(22)
    n = 1024
    Q1, _ = np.linalg.qr(rng.randn(n, n))
    Q2, _ = np.linalg.qr(rng.randn(n, n))
    A = (Q1 * np.logspace(0, 6, n)) @ Q2.T
    b = rng.randn(n)
    xr = np.linalg.solve(A, b)

    def err(x):
        return np.linalg.norm(x - xr) / np.linalg.norm(xr)

    case("solve ozaki n=1024 cond 1e6 without torch")
    x = ozk.solve(A, b, residual_mode="ozaki")
    assert isinstance(x, np.ndarray) and x.shape == (n,)
    e_ref = err(O.solve_ozaki(A, b))
    assert err(x) <= 2.0 * e_ref
    assert e_ref < err(O.solve_ozaki(A, b, max_iterations=0)) / 10.0
    case("solve f64 residuals, 3 right-hand sides, well conditioned, without torch")
    W = rng.randn(n, n) + n * np.eye(n)
    B = rng.randn(n, 3)
    Xs = ozk.solve(W, B)
    assert Xs.shape == (n, 3)
    assert np.linalg.norm(Xs - np.linalg.solve(W, B)) / np.linalg.norm(Xs) < 1e-13
    case("inv n=200 without torch (FP64 and Ozaki residuals)")
    M = rng.randn(200, 200) + 200 * np.eye(200)
    assert np.abs(ozk.inv(M) @ M - np.eye(200)).max() < 1e-13
    Mr = np.linalg.inv(M)
    Mi = ozk.inv(M, residual_mode="ozaki")
    assert np.linalg.norm(Mi - Mr) / np.linalg.norm(Mr) <= 1e-6  # the Tier-1 bound
    case("norms without torch")
    v = rng.randn(300)
    for o in (None, 2, 1, np.inf, -np.inf, 0, 3):
        assert np.isclose(ozk.norm(v, o), np.linalg.norm(v, o), rtol=1e-14)
    G = rng.randn(400, 60)
    for o in (None, "fro", 1, -1, np.inf, -np.inf):
        assert np.isclose(ozk.norm(G, o), np.linalg.norm(G, o), rtol=1e-14)
    s2 = ozk.norm(G, 2, mode="ozaki")
    assert isinstance(s2, np.float64)
    assert np.isclose(s2, np.linalg.norm(G, 2), rtol=1e-12)
