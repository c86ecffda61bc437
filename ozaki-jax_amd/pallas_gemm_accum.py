"""The fused slice-GEMM + 2Sum kernel (mirror of ``ozaki_jax/pallas_gemm_accum.py``).

The reference's Pallas TPU kernel keeps every slice-pair product in VMEM and
returns the double-float pair (C_hi, C_lo).  Here the same computation is
the library's fused all-pairs kernel (pairwise kernel for custom (n_hi,
n_lo)): ozk_gemm_2sum_pair returns the pair, ozk_gemm its FP64 sum.  The
reference's tile sizes (bm, bk, bn) are TPU block shapes; they are accepted
and not used (the kernel's tiling is fixed for gfx950).
"""

import numpy as np

from . import _device as D
from . import _lib
from .lowlevel import unit_swizzle

_CHUNK_BF16 = 32   # BF16 values in one 64-byte chunk of a plane line
_LINE_PAD = 64     # plane lines are padded to a multiple of 64


def _make_pair_schedule(n_hi, n_lo):
    """pallas_gemm_accum.py:26-87: pair indices (hh, hl, lh, i-major),
    groups (A-slice index, pair indices) and block boundaries."""
    n_total = n_hi + n_lo
    pair_a, pair_b = [], []
    for i in range(n_hi):
        for j in range(n_hi):
            pair_a.append(i)
            pair_b.append(j)
    for i in range(n_hi):
        for j in range(n_lo):
            pair_a.append(i)
            pair_b.append(n_hi + j)
    for i in range(n_lo):
        for j in range(n_hi):
            pair_a.append(n_hi + i)
            pair_b.append(j)
    groups, idx = [], 0
    for a, size in ([(i, n_hi) for i in range(n_hi)] + [(i, n_lo) for i in range(n_hi)]
                    + [(n_hi + i, n_hi) for i in range(n_lo)]):
        groups.append((a, tuple(range(idx, idx + size))))
        idx += size
    assert idx == len(pair_a) and n_total == n_hi + n_lo
    return (tuple(pair_a), tuple(pair_b), len(pair_a), tuple(groups),
            (n_hi, 2 * n_hi, 2 * n_hi + n_lo))


def _pack_bf16_planes(lines):
    """(planes, L, K) float32 BF16-exact slice values -> the library's BF16
    plane layout (planes, L padded to 64, K padded to 64), uint16: per plane,
    64-byte chunks of k, chunk c of every line together, the four 16-byte
    units of a line's chunk in the order u ^ unit_swizzle(line)."""
    s = np.ascontiguousarray(np.asarray(lines, dtype=np.float32))
    bits = s.view(np.uint32)
    if np.any(bits & 0xffff):
        raise ValueError("slices must be BF16-exact (as the extraction produces them)")
    n, L, K = s.shape
    Lp = -(-max(L, 1) // _LINE_PAD) * _LINE_PAD
    Kp = -(-max(K, 1) // 64) * 64
    g = np.zeros((n, Lp, Kp), np.uint16)
    g[:, :L, :K] = (bits >> 16).astype(np.uint16)
    nch = Kp // _CHUNK_BF16
    g = g.reshape(n, Lp, nch, 4, 8)
    r = np.arange(Lp)
    stored = np.arange(4)[None, :] ^ unit_swizzle(r)[:, None]       # (Lp, 4)
    g = g[:, r[:, None], :, stored, :]                               # (Lp, 4, n, nch, 8)
    g = g.transpose(2, 3, 0, 1, 4)                                   # (n, nch, Lp, 4, 8)
    return np.ascontiguousarray(g).reshape(n, Lp, Kp), Lp


def _exps(scales, lines_pad):
    e = np.zeros((scales.shape[0], lines_pad), np.int32)
    with np.errstate(invalid="ignore"):
        e[:, :scales.shape[1]] = np.asarray(scales, np.float64).astype(np.int32)
    return e


def fused_gemm_accum(a_slices, b_slices, a_scales, b_scales, n_hi, n_lo, *,
                     bm=128, bk=128, bn=128):
    """pallas_gemm_accum.py:191-275.  a_slices (n_hi + n_lo, N, K) and
    b_slices (n_hi + n_lo, K, M) FP32 BF16-exact slices, a_scales (.., N)
    and b_scales (.., M) their exponents; returns (C_hi, C_lo), FP32 N x M,
    in the family of a_slices."""
    want_torch = D.is_torch(a_slices)

    def host(x):
        return x.detach().cpu().numpy() if D.is_torch(x) else np.asarray(x)

    a, b = host(a_slices), host(b_slices)
    ae, be = host(a_scales), host(b_scales)
    n_total = n_hi + n_lo
    if a.ndim != 3 or b.ndim != 3 or a.shape[0] != n_total or b.shape[0] != n_total:
        raise ValueError("expected (n_hi + n_lo, N, K) and (n_hi + n_lo, K, M) slices")
    if a.shape[2] != b.shape[1]:
        raise ValueError(f"incompatible slice shapes {a.shape} and {b.shape}")
    N, K = a.shape[1], a.shape[2]
    M = b.shape[2]
    fam = D.family(want_torch)
    pa, La = _pack_bf16_planes(a)
    pb, Lb = _pack_bf16_planes(b.transpose(0, 2, 1))
    A_dev = _upload(fam, pa)
    B_dev = _upload(fam, pb)
    Ae_dev, Be_dev = _upload(fam, _exps(ae, La)), _upload(fam, _exps(be, Lb))
    C_hi, C_lo = fam.empty((N, M), np.float32), fam.empty((N, M), np.float32)
    if N and M:
        lib = _lib.load()
        wsb = lib.ozk_gemm_workspace_bytes(N, M, _lib.PIPE_ONDEVICE, n_hi, n_lo,
                                           _lib.ORDER_2SUM)
        ws = fam.workspace(wsb)
        _lib.check(lib.ozk_gemm_2sum_pair(
            A_dev.data_ptr(), Ae_dev.data_ptr(), None, B_dev.data_ptr(), Be_dev.data_ptr(),
            None, N, M, max(K, 1), 2, 0, n_hi, n_lo, C_hi.data_ptr(), C_lo.data_ptr(),
            max(M, 1), ws.data_ptr(), wsb, fam.stream()))
    return fam.out(C_hi, want_torch), fam.out(C_lo, want_torch)


def _upload(fam, a):
    """A host array on the device, in family `fam` (same dtype)."""
    if isinstance(fam, D._HipFamily):
        from ._hip import DeviceArray
        return DeviceArray.from_numpy(a)
    return D.torch.from_numpy(np.ascontiguousarray(a)).to(fam.dev)


def fused_ozaki_matmul(A_f64, B_f64, rho, n_hi, n_lo, *, bm=128, bk=128, bn=128):
    """pallas_gemm_accum.py:278-316: split, FP32 extraction with the given
    rho (A rows, B columns), fused slice GEMMs with 2Sum accumulation, FP64
    combine; returns the FP64 product in A's family."""
    from . import lowlevel as ll
    want_torch = D.is_torch(A_f64)
    fam = D.family(True)  # the stage-level planes are torch tensors
    A = fam.f64(A_f64)
    B = fam.f64(B_f64)
    if A.shape[1] != B.shape[0]:
        raise ValueError(f"incompatible shapes {tuple(A.shape)} and {tuple(B.shape)}")
    pa = ll.extract(A, 0, int(rho), n_hi, n_lo)
    pb = ll.extract(B, 1, int(rho), n_hi, n_lo)
    C = ll.gemm(pa, pb, ll.PIPE_ONDEVICE, n_hi, n_lo, ll.ORDER_2SUM)
    return C if want_torch else C.cpu().numpy()


__all__ = ["fused_gemm_accum", "fused_ozaki_matmul"]
