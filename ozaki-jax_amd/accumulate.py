"""Standalone 2Sum accumulation (mirror of ``accumulate_2sum`` and
``validate_accumulation_2sum`` in ``ozaki_jax/pallas_ops.py``).

accumulate_2sum runs the A4 order (pallas_ops.py:178-239) on products the
caller holds, in the HIP kernel behind ``ozk_accumulate_2sum``.  Every
backend name the reference accepts runs that kernel.
"""

import numpy as np

from . import _device as D
from . import _lib
from . import lowlevel as ll
from .extract import rho_f32

_MAX_PRESET = (5, 4)  # matmul.py:168-172 "max"


def _to_device_f32(x, dev):
    if D.is_torch(x):
        t = x.detach().to(device=dev, dtype=D.torch.float32)
    else:
        t = D.torch.from_numpy(np.ascontiguousarray(np.asarray(x, dtype=np.float32))).to(dev)
    return t.contiguous()


def _accumulate(P, cs, rs, block_group_sizes):
    """(C_hi, C_lo) device tensors from device tensors P (n, N, M), cs (n, M),
    rs (g, N)."""
    lib = _lib.load()
    n_prod, N, M = P.shape
    blocks = [tuple(int(s) for s in b) for b in block_group_sizes]
    ngroups = np.array([len(b) for b in blocks], dtype=np.int32)
    sizes = np.array([s for b in blocks for s in b], dtype=np.int32)
    if sizes.sum() != n_prod:
        raise ValueError(f"block_group_sizes cover {int(sizes.sum())} products, "
                         f"products holds {n_prod}.")
    if cs.shape != (n_prod, M):
        raise ValueError(f"col_scales shape {tuple(cs.shape)} != ({n_prod}, {M}).")
    if rs.shape != (len(sizes), N):
        raise ValueError(f"row_scales shape {tuple(rs.shape)} != ({len(sizes)}, {N}).")
    Ch = D.torch.empty((N, M), dtype=D.torch.float32, device=P.device)
    Cl = D.torch.empty((N, M), dtype=D.torch.float32, device=P.device)
    _lib.check(lib.ozk_accumulate_2sum(
        P.data_ptr(), n_prod, N, M, cs.data_ptr(), rs.data_ptr(),
        ngroups.ctypes.data, len(ngroups), sizes.ctypes.data, len(sizes),
        Ch.data_ptr(), Cl.data_ptr(), D.stream_handle()))
    return Ch, Cl


def accumulate_2sum(products, col_scales, row_scales, block_group_sizes,
                    N=None, M=None, backend="auto"):
    """pallas_ops.py:372-396.  products (n_products, N, M), col_scales
    (n_products, M), row_scales (n_groups, N), FP32; block_group_sizes one
    tuple of group sizes per block.  Returns (C_hi, C_lo), FP32 (N, M), as
    torch tensors for torch input and NumPy arrays otherwise."""
    if backend not in ("pallas", "auto", "jax"):
        raise ValueError(
            f"Unknown backend={backend!r}; expected 'auto', 'jax', or 'pallas'.")
    want_torch = D.is_torch(products)
    dev = D.require_gpu()
    P = _to_device_f32(products, dev)
    if P.dim() != 3:
        raise ValueError(f"products must be 3D (n_products, N, M), got ndim={P.dim()}.")
    Ch, Cl = _accumulate(P, _to_device_f32(col_scales, dev),
                         _to_device_f32(row_scales, dev), block_group_sizes)
    if backend == "pallas":  # the Pallas path strips padding to (N, M)
        n = P.shape[1] if N is None or M is None else N
        m = P.shape[2] if N is None or M is None else M
        Ch, Cl = Ch[:n, :m], Cl[:n, :m]
    return D.to_family(Ch, want_torch), D.to_family(Cl, want_torch)


def _pow2(e):
    """FP32 2^e for an integer exponent tensor e (same shape): the FP64 power
    of two from its bit pattern, rounded to FP32 (exact, and 0 below 2^-149,
    as np.ldexp on float32 gives)."""
    bits = (e.to(D.torch.int64) + 1023) << 52
    return bits.view(D.torch.float64).to(D.torch.float32)


def validate_accumulation_2sum(N=128, M=128, K=128):
    """pallas_ops.py:399-467: 2Sum accumulation of the max preset's products
    against the FP64 block accumulation and the FP64 product, on
    RandomState(42) data.  Extraction, products, the A3 baseline and the 2Sum
    accumulation all run in the HIP kernels."""
    rng = np.random.RandomState(42)
    A = rng.randn(N, K).astype(np.float64)
    B = rng.randn(K, M).astype(np.float64)
    C_exact = A @ B
    n_hi, n_lo = _MAX_PRESET
    rho = rho_f32(K)
    D.require_gpu()
    pa = ll.extract(A, 0, rho, n_hi, n_lo)
    pb = ll.extract(B, 1, rho, n_hi, n_lo)
    P = ll.slice_products(pa, pb, _lib.PIPE_ONDEVICE, n_hi, n_lo)
    C_baseline = ll.gemm(pa, pb, _lib.PIPE_ONDEVICE, n_hi, n_lo,
                         _lib.ORDER_BLOCK64).cpu().numpy()
    baseline_err = float(np.max(np.abs(C_baseline - C_exact)) / np.max(np.abs(C_exact)))

    # pallas_ops.py:105-175: column scales per product (hh, hl, lh), row
    # scales per group, block group sizes.
    # Exponents are per line: (slices, N) for A's rows, (slices, M) for B's
    # columns.
    ae, be = pa.exponents(), pb.exponents()
    a_hi, a_lo = _pow2(ae[:n_hi]), _pow2(ae[n_hi:])
    b_hi, b_lo = _pow2(be[:n_hi]), _pow2(be[n_hi:])
    cs = D.torch.cat([b_hi.repeat(n_hi, 1), b_lo.repeat(n_hi, 1), b_hi.repeat(n_lo, 1)])
    rs = D.torch.cat([a_hi, a_hi, a_lo])
    bgs = (tuple([n_hi] * n_hi), tuple([n_lo] * n_hi), tuple([n_hi] * n_lo))
    Ch, Cl = _accumulate(P.contiguous(), cs.contiguous(), rs.contiguous(), bgs)
    C_2sum = (Ch.to(D.torch.float64) + Cl.to(D.torch.float64)).cpu().numpy()
    twosum_err = float(np.max(np.abs(C_2sum - C_exact)) / np.max(np.abs(C_exact)))
    return {
        "match": twosum_err < 1e-9,
        "max_rel_error": twosum_err,
        "baseline_error": baseline_err,
        "N": N, "M": M, "K": K,
    }


__all__ = ["accumulate_2sum", "validate_accumulation_2sum"]
