"""The double-float pair (C_hi, C_lo) of the 2Sum order
(pallas_gemm_accum.py:181-186, the result of `fused_gemm_accum`), against
the oracle's pair (order A4), bit for bit, and the FP64 combine of
`fused_ozaki_matmul` (pallas_gemm_accum.py:278-316) at a caller's rho."""

import sys

import numpy as np
import pytest

import oracle as O
from oracle import pipeline as OP

pytestmark = pytest.mark.gpu


def case(msg):
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def _oracle_pair(A, B, rho, nh, nl):
    a, ae, b, be = OP.ondevice_slices(A, B, rho, nh, nl)
    sched = OP.ondevice_schedule(nh, nl)
    return (a, ae, b, be), OP.accumulate_a4(OP.slice_products(a, b, sched), sched, ae, be)


@pytest.mark.parametrize("nh,nl", [(4, 1), (3, 1), (5, 4), (2, 3), (4, 2), (5, 1), (6, 1),
                                   (7, 6), (9, 1)])
def test_fused_gemm_accum_pair(ozk, nh, nl):
    """Caller-held slices (the oracle's) through the NumPy family: all-pairs
    kernel for the presets, (2, 3) (one sweep), (4, 2) (two sweeps; the fold
    state crosses the workspace) and (5, 1) (three); rectangle sweeps for
    (6, 1) and (7, 6) (the block sums cross the workspace too); pairwise
    kernel for (9, 1)."""
    from ozaki_jax_amd.pallas_gemm_accum import fused_gemm_accum
    rng = np.random.RandomState(nh * 10 + nl)
    A = (rng.rand(96, 200) - 0.5) * np.exp(2 * rng.randn(96, 200))
    B = rng.randn(200, 70)
    rho = O.rho_f32(200)
    (a, ae, b, be), (ch, cl) = _oracle_pair(A, B, rho, nh, nl)
    case(f"fused_gemm_accum ({nh},{nl}) (96,200,70)")
    hi, lo = fused_gemm_accum(a, b, ae, be, nh, nl)
    assert hi.dtype == np.float32 and lo.dtype == np.float32
    assert np.array_equal(hi, ch) and np.array_equal(lo, cl)
    assert np.array_equal(hi.astype(np.float64) + lo.astype(np.float64),
                          O.matmul_ondevice_a4(A, B, "raise", nh, nl))


@pytest.mark.parametrize("nh,nl", [(4, 1), (5, 4), (4, 2), (6, 1), (8, 8)])
def test_gemm_pair_int8_planes(ozk, nh, nl):
    """INT8 planes (K = 5000 and 4200, rho = 19), 16 and 324 tiles."""
    import torch
    from ozaki_jax_amd import lowlevel as ll
    rng = np.random.RandomState(nh)
    for N, K, M in [(70, 5000, 60), (1100, 4200, 1100)]:
        if nl > 1 and N > 100:
            continue
        A, B = rng.randn(N, K), (rng.rand(K, M) - 0.5) * np.exp(2 * rng.randn(K, M))
        rho = O.rho_f32(K)
        pa = ll.extract(A, 0, rho, nh, nl, i8=True)
        pb = ll.extract(B, 1, rho, nh, nl, i8=True)
        case(f"ozk_gemm_2sum_pair int8 ({nh},{nl}) ({N},{K},{M})")
        hi, lo = ll.gemm_pair(pa, pb, nh, nl)
        rows = np.r_[0:8, N - 8:N]
        _, (ch, cl) = _oracle_pair(A[rows], B, rho, nh, nl)
        assert np.array_equal(hi.cpu().numpy()[rows], ch)
        assert np.array_equal(lo.cpu().numpy()[rows], cl)
        assert isinstance(hi, torch.Tensor)


@pytest.mark.parametrize("nh,nl", [(4, 2), (6, 1)])
def test_gemm_pair_int8_planes_dynamic_tail(ozk, nh, nl):
    """A multi-sweep schedule over 33 x 33 tiles (four whole rounds on 256
    CUs, then the dynamic tail): the pair form keeps the 2Sum fold state in
    the workspace ahead of the tile counters, as the FP64 form does."""
    from ozaki_jax_amd import lowlevel as ll
    rng = np.random.RandomState(40 + nh)
    N, K, M = 2112, 4200, 2112
    A, B = rng.randn(N, K), (rng.rand(K, M) - 0.5) * np.exp(2 * rng.randn(K, M))
    rho = O.rho_f32(K)
    pa = ll.extract(A, 0, rho, nh, nl, i8=True)
    pb = ll.extract(B, 1, rho, nh, nl, i8=True)
    case(f"ozk_gemm_2sum_pair int8 ({nh},{nl}) ({N},{K},{M}) dynamic tail")
    hi, lo = ll.gemm_pair(pa, pb, nh, nl)
    rows = np.r_[0:4, 1055:1059, N - 4:N]
    _, (ch, cl) = _oracle_pair(A[rows], B, rho, nh, nl)
    assert np.array_equal(hi.cpu().numpy()[rows], ch)
    assert np.array_equal(lo.cpu().numpy()[rows], cl)


def test_fused_ozaki_matmul_given_rho(ozk):
    from ozaki_jax_amd.pallas_gemm_accum import fused_ozaki_matmul
    rng = np.random.RandomState(9)
    A, B = rng.randn(80, 300), rng.randn(300, 50)
    for rho, nh, nl in [(20, 4, 1), (17, 3, 1), (22, 5, 4)]:
        case(f"fused_ozaki_matmul rho={rho} ({nh},{nl})")
        C = fused_ozaki_matmul(A, B, rho, nh, nl)
        assert np.array_equal(C, OP._ozaki_a4_unchecked(A, B, rho, nh, nl))
