"""C ABI checks that need no GPU: the library loads, exports every function
declared in include/ozaki_amd.h with the bound signature, its host-only
functions agree with the oracle, and invalid arguments are rejected before
any device work (no compute calls are made here)."""

import ctypes
import re

import numpy as np
import pytest

import oracle as O
from conftest import ROOT

HEADER = ROOT / "include" / "ozaki_amd.h"


@pytest.fixture(scope="module")
def lib():
    from ozaki_jax_amd import _lib
    return _lib.load()


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(ozk_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    from ozaki_jax_amd import _lib
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(str(ROOT / "ozaki-jax_amd" / "libozaki_amd.so"))
    for name in declared_functions():
        assert hasattr(raw, name), name


def test_header_compiles_as_c(tmp_path):
    import subprocess
    src = tmp_path / "t.c"
    src.write_text('#include "ozaki_amd.h"\nint main(void){return ozk_abi_version() < 0;}\n')
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-c", str(src),
                    "-I", str(ROOT / "include"), "-o", str(tmp_path / "t.o")],
                   check=True)


def test_host_functions(lib):
    assert lib.ozk_abi_version() == 3
    for K in [1, 2, 3, 64, 1040, 4096, 8192, 32768, 65536, 2 ** 22, 2 ** 22 + 1, 10 ** 9]:
        assert lib.ozk_rho_f32(K) == O.rho_f32(K)
        assert lib.ozk_rho_f64(K) == O.rho_f64(K)
    assert lib.ozk_slice_ld(1) == 64 and lib.ozk_slice_ld(65) == 128
    assert lib.ozk_slice_lines(8192) == 8192
    assert lib.ozk_pair_count(0, 4, 1) == 24
    assert lib.ozk_pair_count(0, 5, 4) == 65
    assert lib.ozk_pair_count(1, 8, 0) == 36
    assert lib.ozk_pair_count(0, 0, 1) == -1
    assert b"outside" in lib.ozk_last_error()


# dynamic-tail words of an all-pairs product: 64 counters and one word per
# workgroup (up to 1024)
DYN = (128 + 1024) * 4


def r256(b):
    return -(-b // 256) * 256


def gang_bytes(rows, cols):
    """Column extraction of 4097 to 65536 rows on the FP32 path: the ticket
    word and, per 16-column panel, the exchange records of up to 32 rounds
    for each 512-row run of a column (32 words a round, 128 in round 1;
    256-byte aligned).  The members add their INT8 line sums into the
    plane sums directly.  Columns of up to 4096 rows need no workspace."""
    ld = -(-rows // 64) * 64
    if ld <= 4096:
        return 0
    G = -(-ld // 512)
    lp = -(-cols // 64) * 64
    return r256(256 + (lp // 16) * G * (32 + 128 + 30 * 32) * 4)


def row_gang_bytes(lines, length):
    """FP32 lines of 32769 to 262144 elements: the ticket word and, per
    (line, slice) for up to 32 slices, one 128-byte exchange record
    (256-byte aligned).  The members add their INT8 line sums into the plane
    sums directly."""
    lp = -(-lines // 64) * 64
    return r256(256 + lp * 32 * 128)


def test_workspace_sizes(lib):
    # A and B slice planes + exponents (+ line sums on INT8 planes) + B's
    # column-extraction exchange records; planes are INT8 when K > 4096
    # (rho >= 19) and the schedule is a preset, else BF16
    for K, eb in [(8192, 1), (4096, 2)]:
        N = M = 8192
        for nh, nl in [(4, 1), (3, 1)]:
            ws = lib.ozk_matmul_workspace_bytes(N, K, M, 0, nh, nl)
            planes = 2 * (nh + nl) * 8192 * K * eb
            extra = (2 if eb == 1 else 1) * 2 * (nh + nl) * 8192 * 4 + 4096 + DYN
            assert planes + gang_bytes(K, M) <= ws <= planes + gang_bytes(K, M) + extra, (K, nh, nl)
    # max (5, 4): INT8 planes + exchange records + the 2Sum fold state
    # between its three sweeps (5 FP32 fields per output element)
    ws = lib.ozk_matmul_workspace_bytes(8192, 8192, 8192, 0, 5, 4)
    base = 2 * 9 * 8192 * 8192 + gang_bytes(8192, 8192) + 20 * 8192 * 8192
    assert base <= ws <= base + 2 * 2 * 9 * 8192 * 4 + 8192 + DYN
    # columns longer than 65536 rows, and the FP64 (host) pipeline, transpose
    # B; one extraction buffer serves A's rows and B's columns in turn
    ws = lib.ozk_matmul_workspace_bytes(64, 70000, 64, 0, 4, 1)
    assert ws >= 8 * 70000 * 64 + row_gang_bytes(64, 70000)
    N, K, M = 1024, 65536, 1024
    ws = lib.ozk_matmul_workspace_bytes(N, K, M, 0, 4, 1)
    planes = 5 * (N + M) * K + 2 * 5 * (N + M) * 4
    ex = max(row_gang_bytes(N, K), gang_bytes(K, M))
    assert planes + ex <= ws <= planes + ex + 4096 + DYN
    assert ws - planes < 8 * K * M  # no transposed copy of B
    ws = lib.ozk_matmul_workspace_bytes(64, 1000, 64, 1, 8, 0)
    assert ws >= 8 * 1000 * 64


def test_residual_workspace_bytes(lib):
    # the fused row kernels need no workspace: high / medium up to K = 16384,
    # max up to 8192, up to 4 right-hand sides; other cases take the
    # slice-GEMM route and its workspace
    for nh, nl, kmax in ((4, 1, 16384), (3, 1, 16384), (5, 4, 8192)):
        for K in (1, 700, 1024, 1025, 2049, kmax):
            assert lib.ozk_residual_workspace_bytes(300, K, 1, nh, nl) == 0, (nh, nl, K)
        assert lib.ozk_residual_workspace_bytes(300, kmax, 4, nh, nl) == 0
        assert lib.ozk_residual_workspace_bytes(300, kmax + 1, 1, nh, nl) > 0
        assert lib.ozk_residual_workspace_bytes(300, 700, 5, nh, nl) > 0
    assert lib.ozk_residual_workspace_bytes(300, 700, 1, 4, 2) > 0


def test_gemm_workspace_bytes(lib):
    # all-pairs schedules: the fold state the three-sweep max schedule keeps
    # between launches (rounded to 256 B), then the dynamic-tail words (8
    # counters for each of up to 16 sweeps and one word for each of up to
    # 1024 workgroups)
    dyn = DYN

    def up(x):
        return (x + 255) // 256 * 256

    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 4, 1, 0) == dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 3, 1, 1) == dyn
    # host schedules of up to 9 slices: all-pairs sweeps over groups of A
    # planes (one for up to 5 slices; 8 slices take three, 9 four, with the
    # FP64 running sum kept between them); more slices run the pairwise kernel
    assert lib.ozk_gemm_workspace_bytes(100, 70, 1, 8, 0, 3) == up(100 * 70 * 8) + dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 1, 5, 0, 2) == dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 1, 9, 0, 3) == up(100 * 70 * 8) + dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 1, 10, 0, 3) == 0
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 5, 4, 0) == up(100 * 70 * 20) + dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 5, 4, 1) == up(100 * 70 * 8) + dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 5, 4, -1) == dyn
    # on-device schedules beyond (5, 5), both counts up to 8: rectangle
    # sweeps; where one cuts a block the 2Sum state also carries the block's
    # running sum (7 FP32 fields).  (6, 1): hh in two sweeps of 3 groups;
    # (1, 6): one sweep per block.  Per-pair products and larger counts run
    # the pairwise kernel.
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 6, 1, 0) == up(100 * 70 * 28) + dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 6, 1, 1) == up(100 * 70 * 8) + dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 1, 6, 0) == up(100 * 70 * 20) + dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 8, 8, 0) == up(100 * 70 * 28) + dyn
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 6, 1, -1) == 0
    assert lib.ozk_gemm_workspace_bytes(100, 70, 0, 9, 1, 0) == 0
    assert lib.ozk_extract_workspace_bytes(100, 50, 0) == 0
    assert lib.ozk_extract_workspace_bytes(100, 32768, 0) == 0
    # rows of 32769 to 262144 elements: row gangs; longer lines stream
    assert lib.ozk_extract_workspace_bytes(3, 32769, 0) == row_gang_bytes(3, 32769)
    assert lib.ozk_extract_workspace_bytes(100, 262144, 0) == row_gang_bytes(100, 262144)
    assert lib.ozk_extract_workspace_bytes(3, 262145, 0) == 0
    # the larger of the FP32 (none for columns of up to 4096 rows, else the
    # exchange records) and FP64 (transpose, rounded up to 256 bytes) needs
    assert lib.ozk_extract_workspace_bytes(100, 50, 1) == 40192
    assert lib.ozk_extract_workspace_bytes(8, 5000, 1) == 320000
    assert lib.ozk_extract_workspace_bytes(5000, 8, 1) == max(320000, gang_bytes(5000, 8))
    assert lib.ozk_extract_workspace_bytes(5000, 1, 1) == gang_bytes(5000, 1) > 40000
    # longer columns: the transposed copy (256-byte aligned), then the row
    # gangs' records while the transposed lines are within their reach
    assert lib.ozk_extract_workspace_bytes(70000, 3, 1) == 1680128 + row_gang_bytes(3, 70000)
    assert lib.ozk_extract_workspace_bytes(300000, 3, 1) == 300000 * 3 * 8


def test_int8_entry_points_reject_before_device_work(lib):
    from ozaki_jax_amd import _lib
    # INT8 planes need 19 <= rho <= 24 (|q| <= 64, stored with an offset of
    # at most 63) and an all-pairs schedule: every (n_hi, n_lo) with both
    # counts in 1 .. 8; others, such as (9,1), (1,9) and (9,9), run on BF16
    # planes.  Per-pair products of INT8 planes: counts up to 5.
    for rho in (18, 25):
        rc = lib.ozk_extract_f32_i8(None, 4, 4, 4, 0, rho, 4, 1, None, None, None, None, None,
                                    0, None)
        assert rc == _lib.OZK_ERR_UNSUPPORTED and b"19 <= rho <= 24" in lib.ozk_last_error()
        rc = lib.ozk_gemm_i8(None, None, None, None, None, None, 4, 4, 8192, rho, 4, 1, 0,
                             None, 4, None, 0, None)
        assert rc == _lib.OZK_ERR_UNSUPPORTED
    for nh, nl in ((9, 1), (1, 9), (9, 9)):
        rc = lib.ozk_gemm_i8(None, None, None, None, None, None, 4, 4, 8192, 19, nh, nl, 0,
                             None, 4, None, 0, None)
        assert rc == _lib.OZK_ERR_UNSUPPORTED and b"all-pairs" in lib.ozk_last_error()
        rc = lib.ozk_slice_products_i8(None, None, None, None, 4, 4, 8192, 19, nh, nl, None, 4,
                                       None)
        assert rc == _lib.OZK_ERR_UNSUPPORTED
    for nh, nl in ((6, 1), (8, 8)):
        rc = lib.ozk_slice_products_i8(None, None, None, None, 4, 4, 8192, 19, nh, nl, None, 4,
                                       None)
        assert rc == _lib.OZK_ERR_UNSUPPORTED and b"fixed all-pairs" in lib.ozk_last_error()
    rc = lib.ozk_gemm_i8(None, None, None, None, None, None, 4, 4, 8192, 19, 4, 1, 7, None, 4,
                         None, 0, None)
    assert rc == _lib.OZK_ERR_INVALID
    # the line sums are required
    rc = lib.ozk_gemm_i8(None, None, None, None, None, None, 4, 4, 8192, 19, 4, 1, 0, None, 4,
                         None, 0, None)
    assert rc == _lib.OZK_ERR_INVALID and b"null pointer" in lib.ozk_last_error()
    rc = lib.ozk_slice_products_i8(None, None, None, None, 4, 4, 8192, 19, 4, 1, None, 4, None)
    assert rc == _lib.OZK_ERR_INVALID


def test_argument_errors_before_device_work(lib):
    from ozaki_jax_amd import _lib
    # bad slice counts / order / shapes are rejected with OZK_ERR_INVALID and
    # a message; no pointer is dereferenced and no kernel is launched.
    rc = lib.ozk_gemm(None, None, None, None, 4, 4, 4, 0, 0, 1, 0, None, 4, None, 0, None)
    assert rc == _lib.OZK_ERR_INVALID
    rc = lib.ozk_gemm(None, None, None, None, 4, 4, 4, 0, 4, 1, 9, None, 4, None, 0, None)
    assert rc == _lib.OZK_ERR_INVALID and b"order" in lib.ozk_last_error()
    rc = lib.ozk_matmul(None, 4, None, 4, None, 4, 4, 0, 4, 0, 4, 1, 0, None, 0, None, None)
    assert rc == _lib.OZK_ERR_INVALID and b"invalid shape" in lib.ozk_last_error()
    rc = lib.ozk_matmul(None, 2, None, 4, None, 4, 4, 4, 4, 0, 4, 1, 0, None, 0, None, None)
    assert rc == _lib.OZK_ERR_INVALID and b"leading dimension" in lib.ozk_last_error()
    rc = lib.ozk_extract_f32(None, 4, 4, 4, 0, 19, 40, 1, None, None, None, None, 0, None)
    assert rc == _lib.OZK_ERR_INVALID
    rc = lib.ozk_gram(None, 4, 0, 4, 4, 1, None, 4, None, 0, None, None)
    assert rc == _lib.OZK_ERR_INVALID
    with pytest.raises(ValueError):
        _lib.check(rc)
    # the early-flag variants check their host word and event first
    rc = lib.ozk_matmul_early_flags(None, 4, None, 4, None, 4, 4, 4, 4, 0, 4, 1, 0, None, 0,
                                    None, None, None, None)
    assert rc == _lib.OZK_ERR_INVALID and b"host flag word" in lib.ozk_last_error()
    rc = lib.ozk_gram_early_flags(None, 4, 4, 4, 4, 1, None, 4, None, 0, None, None, None,
                                  None)
    assert rc == _lib.OZK_ERR_INVALID and b"host flag word" in lib.ozk_last_error()
    # and then the same arguments as ozk_matmul / ozk_gram
    word = (ctypes.c_uint32 * 1)()
    rc = lib.ozk_matmul_early_flags(None, 4, None, 4, None, 4, 4, 0, 4, 0, 4, 1, 0, None, 0,
                                    None, ctypes.addressof(word), 1, None)
    assert rc == _lib.OZK_ERR_INVALID and b"invalid shape" in lib.ozk_last_error()
    rc = lib.ozk_gram_early_flags(None, 4, 0, 4, 4, 1, None, 4, None, 0, None,
                                  ctypes.addressof(word), 1, None)
    assert rc == _lib.OZK_ERR_INVALID and b"invalid shape" in lib.ozk_last_error()


def test_pivots_to_perm(lib):
    """LAPACK's sequential swaps -> the permutation: row i of P A is row
    perm[i] of A, pinned by P A = L U on SciPy's float64 factors."""
    import scipy.linalg as sla
    from ozaki_jax_amd import _lib
    rng = np.random.RandomState(0)
    for n in (1, 2, 7, 64, 300):
        A = rng.randn(n, n)
        lu, piv = sla.lu_factor(A)
        ipiv = (piv + 1).astype(np.int32)
        perm = np.empty(n, np.int32)
        assert lib.ozk_pivots_to_perm(ipiv.ctypes.data, n, perm.ctypes.data) == 0
        assert sorted(perm) == list(range(n))
        L = np.tril(lu, -1) + np.eye(n)
        U = np.triu(lu)
        assert np.allclose(A[perm], L @ U, rtol=0, atol=1e-12 * n)
    bad = np.array([2, 1], np.int32)  # step 1 swapping with row 0 < 1
    perm = np.empty(2, np.int32)
    assert lib.ozk_pivots_to_perm(bad.ctypes.data, 2, perm.ctypes.data) == _lib.OZK_ERR_INVALID
    assert b"outside" in lib.ozk_last_error()


def test_lu_factor_limits(lib):
    from ozaki_jax_amd import _lib
    nmax = lib.ozk_lu_factor_max_n()
    assert nmax == 4096
    assert lib.ozk_lu_factor_workspace_bytes(0) == 0
    assert lib.ozk_lu_factor_workspace_bytes(nmax) > 0
    flags = ctypes.c_uint32(0)
    rc = lib.ozk_lu_factor_f32(None, nmax + 1, nmax + 1, None, None, 0,
                               ctypes.addressof(flags), None)
    assert rc == _lib.OZK_ERR_UNSUPPORTED and b"panel" in lib.ozk_last_error()
    rc = lib.ozk_lu_factor_f32(None, 3, 4, None, None, 0, ctypes.addressof(flags), None)
    assert rc == _lib.OZK_ERR_INVALID and b"leading dimension" in lib.ozk_last_error()


def test_lu_solve_argument_errors(lib):
    from ozaki_jax_amd import _lib
    assert lib.ozk_lu_solve_workspace_bytes(0, 1) == 0
    assert lib.ozk_lu_solve_workspace_bytes(4096, 3) == 2 * 4096 * 3 * 8
    rc = lib.ozk_lu_solve_f32(None, 4, None, -1, None, 1, None, 1, 1, None, 0, None, None)
    assert rc == _lib.OZK_ERR_INVALID and b"invalid shape" in lib.ozk_last_error()
    rc = lib.ozk_lu_solve_f32(None, 2, None, 4, None, 1, None, 1, 1, None, 0, None, None)
    assert rc == _lib.OZK_ERR_INVALID and b"leading dimension" in lib.ozk_last_error()
    rc = lib.ozk_lu_solve_f32(None, 4, None, 4, None, 1, None, 1, 1, None, 0, None, None)
    assert rc == _lib.OZK_ERR_INVALID and b"flags" in lib.ozk_last_error()


def test_package_fails_loudly_without_gpu():
    import numpy as np
    import torch
    import ozaki_jax_amd as ozk
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(RuntimeError, match="no CPU implementation"):
        ozk.matmul(np.eye(4), np.eye(4), pipeline="ondevice")


@pytest.mark.parametrize("eb,lines,ld", [(1, 64, 64), (1, 128, 192), (2, 64, 64), (2, 192, 128)])
def test_plane_layout_decode_matches_header_formula(eb, lines, ld):
    """Planes.grid() inverts the chunk-major byte layout documented in
    include/ozaki_amd.h: byte b of line r at ((b/64) L + r) 64 +
    16 (((b%64)/16) ^ s(r)) + b%16."""
    import torch
    from ozaki_jax_amd.lowlevel import Planes
    rng = np.random.RandomState(eb * 1000 + lines)
    P = 2
    dt = np.int8 if eb == 1 else np.int16
    grid = rng.randint(-100, 100, size=(P, lines, ld)).astype(dt)
    gb = grid.view(np.uint8).reshape(P, lines, ld * eb)
    store = np.zeros((P, lines * ld * eb), np.uint8)
    for r in range(lines):
        s = (((r & 15) >> 1) ^ ((r & 15) >> 2)) & 3
        for b in range(ld * eb):
            off = ((b // 64) * lines + r) * 64 + 16 * (((b % 64) // 16) ^ s) + b % 16
            store[:, off] = gb[:, r, b]
    st = torch.from_numpy(store.view(dt).reshape(P, lines, ld).copy())
    pl = Planes(st, None, lines, ld, None, rho=19 if eb == 1 else None)
    assert np.array_equal(pl.grid().numpy(), grid)


def test_check_flags_raises_on_wait_timeout():
    from ozaki_jax_amd import _lib
    assert _lib.check_flags(0) == 0
    assert _lib.check_flags(_lib.OZK_FLAG_NONFINITE) == _lib.OZK_FLAG_NONFINITE
    with pytest.raises(RuntimeError, match="OZK_FLAG_WAIT_TIMEOUT"):
        _lib.check_flags(_lib.OZK_FLAG_WAIT_TIMEOUT | _lib.OZK_FLAG_NONFINITE)
