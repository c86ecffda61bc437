"""Ozaki pipelines restated in NumPy (test infrastructure only).

Restates the NumPy-reachable arithmetic of ``ozaki_jax/matmul.py``,
``ozaki_jax/pallas_ops.py`` (accumulation order), ``ozaki_jax/gram.py`` and
``ozaki_jax/solve.py``.  Four accumulation orders exist in the reference; each
is restated once here and named after the reference call site:

  A1  matmul_numpy(pipeline="host") inline loop        matmul.py:879-898
  A2  matmul(pipeline="host") `_accumulate_products`  matmul.py:35-64
  A3  `_accumulate_block_products` (FP64 host accum.)  matmul.py:543-597
  A4  `_accumulate_2sum_logic` double-float 2Sum       pallas_ops.py:178-239
      (== matmul.py:418-488 bf16_interleaved, == pallas_gemm_accum.py:132-186)

Slice indices follow pallas_gemm_accum.py:26-87: A slices 0..n_hi-1 are the
hi-part slices, n_hi..n_hi+n_lo-1 the lo-part slices; the same for B.
"""

import numpy as np

from .extract import (rho_f64, rho_f32, extract_rows_f64, extract_cols_f64,
                      extract_rows_f32, extract_cols_f32)

# matmul.py:168-172
PRECISION_PRESETS = {"high": (4, 1), "medium": (3, 1), "max": (5, 4)}


def resolve_precision(precision):
    """matmul.py:175-194."""
    if isinstance(precision, tuple) and len(precision) == 2:
        n_hi, n_lo = precision
        if n_hi < 1 or n_lo < 1:
            raise ValueError(
                f"Custom precision tuple must have n_hi >= 1 and n_lo >= 1, "
                f"got ({n_hi}, {n_lo}).")
        return precision
    if precision not in PRECISION_PRESETS:
        raise ValueError(
            f"Unknown precision={precision!r}; expected one of "
            f"{sorted(PRECISION_PRESETS)} or a (n_hi, n_lo) tuple.")
    return PRECISION_PRESETS[precision]


def split_hi_lo(X):
    """matmul.py:197-201: hi = f32(x), lo = f32(x - f64(hi))."""
    X = np.asarray(X, dtype=np.float64)
    hi = X.astype(np.float32)
    lo = (X - hi.astype(np.float64)).astype(np.float32)
    return hi, lo


# ---------------------------------------------------------------- schedules

class Schedule:
    """Pair order + group/block structure of one accumulation.

    pair_a[p], pair_b[p]: A / B slice of pair p.
    groups: list of (a_slice, [pairs]) in accumulation order.
    blocks: list of lists of group indices (pallas_gemm_accum.py:81-85).
    """

    def __init__(self, pair_a, pair_b, groups, blocks):
        self.pair_a = list(pair_a)
        self.pair_b = list(pair_b)
        self.groups = groups
        self.blocks = blocks

    @property
    def n_pairs(self):
        return len(self.pair_a)


def ondevice_schedule(n_hi, n_lo):
    """pallas_gemm_accum.py:26-87 / pallas_ops.py:117-173: hh, hl, lh."""
    pa, pb, groups, blocks = [], [], [], []
    specs = [
        [(i, [(i, j) for j in range(n_hi)]) for i in range(n_hi)],            # hh
        [(i, [(i, n_hi + j) for j in range(n_lo)]) for i in range(n_hi)],     # hl
        [(n_hi + i, [(n_hi + i, j) for j in range(n_hi)]) for i in range(n_lo)],  # lh
    ]
    for blk in specs:
        gids = []
        for a, prs in blk:
            idx = []
            for (x, y) in prs:
                idx.append(len(pa))
                pa.append(x)
                pb.append(y)
            gids.append(len(groups))
            groups.append((a, idx))
        blocks.append(gids)
    return Schedule(pa, pb, groups, blocks)


def host_schedule(n_slices):
    """matmul.py:23-32 / :879-883: pairs (i, j) with i + j <= n - 1, i-major."""
    pa, pb, groups = [], [], []
    for i in range(n_slices):
        idx = []
        for j in range(n_slices - i):
            idx.append(len(pa))
            pa.append(i)
            pb.append(j)
        groups.append((i, idx))
    return Schedule(pa, pb, groups, [list(range(len(groups)))])


# ---------------------------------------------------------------- preflight

def _validate_shapes(A, B):
    """matmul.py:67-74."""
    if A.ndim != 2 or B.ndim != 2:
        raise ValueError("Inputs must be rank-2 matrices.")
    if A.shape[1] != B.shape[0]:
        raise ValueError(
            f"Incompatible shapes for matmul: {A.shape} and {B.shape}.")


def _kbound_reasons(K, bits, what):
    reasons = []
    if bits <= 0:
        reasons.append(f"non-positive bits per slice ({bits}); K={K} is too "
                       + what)
    elif K * (2 ** bits - 1) ** 2 >= 2 ** 24:
        max_K = int(2 ** 24 / (2 ** bits - 1) ** 2)
        reasons.append(f"K={K} violates BF16->FP32 exact inner-product bound "
                       f"(need K <= {max_K})")
    return reasons


def host_safety_report(A, B, n_slices):
    """matmul.py:77-116."""
    if n_slices < 1:
        raise ValueError("n_slices must be >= 1.")
    _validate_shapes(A, B)
    K = A.shape[1]
    rho = rho_f64(K)
    bits = 53 - rho
    reasons = _kbound_reasons(
        K, bits, "large for this BF16->FP32 exactness model")
    if n_slices * max(bits, 0) < 53:
        reasons.append(f"insufficient slice budget: n_slices*bits_per_slice="
                       f"{n_slices * max(bits, 0)} < 53")
    if not np.isfinite(A).all() or not np.isfinite(B).all():
        reasons.append("inputs contain NaN or Inf")
    return {"safe": not reasons, "rho": rho, "bits_per_slice": bits,
            "reasons": reasons}


def ondevice_safety_report(A, B, n_hi, n_lo):
    """matmul.py:600-638."""
    _validate_shapes(A, B)
    K = A.shape[1]
    rho = rho_f32(K)
    bits = 24 - rho
    reasons = _kbound_reasons(K, bits, "large for FP32 extraction")
    if not np.isfinite(A).all() or not np.isfinite(B).all():
        reasons.append("inputs contain NaN or Inf")
    return {"safe": not reasons, "rho": rho, "bits_per_slice": bits,
            "n_hi": n_hi, "n_lo": n_lo,
            "n_gemms": n_hi * n_hi + n_hi * n_lo + n_lo * n_hi,
            "reasons": reasons}


def handle_unsafe(A, B, report, safe_mode):
    """matmul.py:119-135: None when safe, A @ B on fallback, else raise."""
    allowed = {"raise", "fallback"}
    if safe_mode not in allowed:
        raise ValueError(f"Invalid safe_mode={safe_mode!r}; expected one of "
                         f"{sorted(allowed)}.")
    if report["safe"]:
        return None
    if safe_mode == "fallback":
        return A @ B
    raise ValueError("Ozaki preflight marked this input as unsafe: "
                     + "; ".join(report["reasons"]))


# ---------------------------------------------------------------- slices

def ondevice_slices(A, B, rho, n_hi, n_lo):
    """matmul.py:745-752: split, then FP32 extraction of the four parts.

    Returns (A_sl (n_t, N, K) f32, A_e (n_t, N) f32,
             B_sl (n_t, K, M) f32, B_e (n_t, M) f32).
    """
    A_hi, A_lo = split_hi_lo(A)
    B_hi, B_lo = split_hi_lo(B)
    ah, ahe = extract_rows_f32(A_hi, rho, n_hi)
    al, ale = extract_rows_f32(A_lo, rho, n_lo)
    bh, bhe = extract_cols_f32(B_hi, rho, n_hi)
    bl, ble = extract_cols_f32(B_lo, rho, n_lo)
    return (np.concatenate([ah, al]), np.concatenate([ahe, ale]),
            np.concatenate([bh, bl]), np.concatenate([bhe, ble]))


def host_slices(A, B, rho, n_slices):
    """matmul.py:875-876: FP64 extraction of A rows and B columns."""
    a, ae = extract_rows_f64(A, rho, n_slices)
    b, be = extract_cols_f64(B, rho, n_slices)
    return a, ae, b, be


def slice_products(A_sl, B_sl, sched):
    """Per-pair FP32 products, as the reference forms them (matmul.py:757-773,
    :885-887): np.float32(a_f32 @ b_f32).  Exact whenever every partial sum
    stays below 2^24 grid units (see products_exact_certificate)."""
    N, M = A_sl.shape[1], B_sl.shape[2]
    P = np.empty((sched.n_pairs, N, M), dtype=np.float32)
    for p in range(sched.n_pairs):
        P[p] = np.float32(A_sl[sched.pair_a[p]].astype(np.float32)
                          @ B_sl[sched.pair_b[p]].astype(np.float32))
    return P


def products_exact_certificate(A_sl, B_sl, sched, unit_a, unit_b):
    """True when, for every pair and output element, the sum of the positive
    terms a_k b_k and the sum of the negative ones both stay below 2^24 grid
    units.  Every partial sum in any summation order lies between those two
    sums, so each is an integer multiple of the grid below 2^24 units and
    exactly representable in FP32: any order gives the same bits.  (The
    terms are integers in grid units, so the FP64 sums below are exact.)"""
    for p in range(sched.n_pairs):
        a = A_sl[sched.pair_a[p]].astype(np.float64) / unit_a
        b = B_sl[sched.pair_b[p]].astype(np.float64) / unit_b
        ap, an = np.maximum(a, 0.0), np.maximum(-a, 0.0)
        bp, bn = np.maximum(b, 0.0), np.maximum(-b, 0.0)
        pos = ap @ bp + an @ bn
        neg = ap @ bn + an @ bp
        if max(pos.max(initial=0.0), neg.max(initial=0.0)) >= 2.0 ** 24:
            return False
    return True


def scales_f32(exps):
    """2^c in FP32 (pallas_ops.py:126-164, matmul.py:276-277)."""
    e = np.asarray(exps)
    return np.ldexp(np.ones(e.shape, dtype=np.float32), e.astype(np.int32))


def scales_f64(exps):
    """2^c in FP64 (matmul.py:42-45, :553-556, :891-894)."""
    e = np.asarray(exps)
    return np.ldexp(np.ones(e.shape, dtype=np.float64), e.astype(np.int64))


# ---------------------------------------------------------------- orders

def _twosum(s, l, x):
    """pallas_ops.py:195-199: t = s + x; e = (s - t) + x; (t, l + e), FP32."""
    t = (s + x).astype(np.float32)
    e = ((s - t).astype(np.float32) + x).astype(np.float32)
    return t, (l + e).astype(np.float32)


def accumulate_a4(P, sched, A_e, B_e):
    """pallas_ops.py:178-239 (order A4).  Returns (C_hi, C_lo) FP32."""
    N, M = P.shape[1], P.shape[2]
    cs = scales_f32(B_e)            # (n_b, M)
    rs = scales_f32(A_e)            # (n_a, N)
    z = np.zeros((N, M), np.float32)
    blk_res = []
    for gids in sched.blocks:
        bh, bl = z.copy(), z.copy()
        for g in gids:
            a, prs = sched.groups[g]
            ih, il = z.copy(), z.copy()
            for p in prs:
                x = (P[p] * cs[sched.pair_b[p]][None, :]).astype(np.float32)
                ih, il = _twosum(ih, il, x)
            r = rs[a][:, None]
            ih = (ih * r).astype(np.float32)
            il = (il * r).astype(np.float32)
            bh, bl = _twosum(bh, bl, ih)
            bh, bl = _twosum(bh, bl, il)
        blk_res.append((bh, bl))
    ch, cl = z.copy(), z.copy()
    for bh, _ in blk_res:
        ch, cl = _twosum(ch, cl, bh)
    for _, bl in blk_res:
        ch, cl = _twosum(ch, cl, bl)
    return ch, cl


def precompute_accumulation_scales(A_hi_e, A_lo_e, B_hi_e, B_lo_e, N, M, n_hi, n_lo):
    """pallas_ops.py:105-175: FP32 column scales per product (schedule order
    hh, hl, lh), row scales per group, and the block/group sizes."""
    def s32(e, n):
        return np.ldexp(np.ones(n, np.float32), np.asarray(e).astype(np.int32))
    cols = ([s32(B_hi_e[j], M) for i in range(n_hi) for j in range(n_hi)]
            + [s32(B_lo_e[j], M) for i in range(n_hi) for j in range(n_lo)]
            + [s32(B_hi_e[j], M) for i in range(n_lo) for j in range(n_hi)])
    rows = ([s32(A_hi_e[i], N) for i in range(n_hi)]
            + [s32(A_hi_e[i], N) for i in range(n_hi)]
            + [s32(A_lo_e[i], N) for i in range(n_lo)])
    bgs = (tuple([n_hi] * n_hi), tuple([n_lo] * n_hi), tuple([n_hi] * n_lo))
    return np.stack(cols), np.stack(rows), bgs


def accumulate_2sum(products, col_scales, row_scales, block_group_sizes):
    """pallas_ops.py:178-239 on explicit arrays: products (P, N, M),
    col_scales (P, M), row_scales (G, N), block_group_sizes a tuple of
    per-block group sizes.  Returns (C_hi, C_lo) FP32."""
    P = np.asarray(products, np.float32)
    cs = np.asarray(col_scales, np.float32)
    rs = np.asarray(row_scales, np.float32)
    N, M = P.shape[1], P.shape[2]
    z = np.zeros((N, M), np.float32)
    blk_res = []
    p = g = 0
    for sizes in block_group_sizes:
        bh, bl = z.copy(), z.copy()
        for size in sizes:
            ih, il = z.copy(), z.copy()
            for _ in range(size):
                ih, il = _twosum(ih, il, (P[p] * cs[p][None, :]).astype(np.float32))
                p += 1
            r = rs[g][:, None]
            ih = (ih * r).astype(np.float32)
            il = (il * r).astype(np.float32)
            bh, bl = _twosum(bh, bl, ih)
            bh, bl = _twosum(bh, bl, il)
            g += 1
        blk_res.append((bh, bl))
    ch, cl = z.copy(), z.copy()
    for bh, _ in blk_res:
        ch, cl = _twosum(ch, cl, bh)
    for _, bl in blk_res:
        ch, cl = _twosum(ch, cl, bl)
    return ch, cl


def combine_f64(ch, cl):
    """matmul.py:526, :540: f64(C_hi) + f64(C_lo)."""
    return ch.astype(np.float64) + cl.astype(np.float64)


def accumulate_a3(P, sched, A_e, B_e):
    """matmul.py:543-597 (order A3): FP32 column scale, FP64 group sum,
    FP64 row scale, FP64 running total over groups in schedule order."""
    N, M = P.shape[1], P.shape[2]
    cs = scales_f32(B_e)
    rs = scales_f64(A_e)
    C = np.zeros((N, M), np.float64)
    for gids in sched.blocks:
        for g in gids:
            a, prs = sched.groups[g]
            inner = np.zeros((N, M), np.float64)
            for p in prs:
                buf = (P[p] * cs[sched.pair_b[p]][None, :]).astype(np.float32)
                inner += buf
            inner *= rs[a][:, None]
            C += inner
    return C


def accumulate_a2(P, sched, A_e, B_e):
    """matmul.py:35-64 (order A2): FP64 column scale, FP64 group sum."""
    N, M = P.shape[1], P.shape[2]
    cs = scales_f64(B_e)
    rs = scales_f64(A_e)
    C = np.zeros((N, M), np.float64)
    for a, prs in sched.groups:
        inner = np.zeros((N, M), np.float64)
        for p in prs:
            buf = P[p].astype(np.float64)
            buf *= cs[sched.pair_b[p]][None, :]
            inner += buf
        inner *= rs[a][:, None]
        C += inner
    return C


def accumulate_a1(P, sched, A_e, B_e):
    """matmul.py:879-898 (order A1): per pair (f64(P) * row) * col, C += ."""
    N, M = P.shape[1], P.shape[2]
    cs = scales_f64(B_e)
    rs = scales_f64(A_e)
    C = np.zeros((N, M), np.float64)
    for p in range(sched.n_pairs):
        t = P[p].astype(np.float64)
        t *= rs[sched.pair_a[p]][:, None]
        t *= cs[sched.pair_b[p]][None, :]
        C += t
    return C


# ---------------------------------------------------------------- drivers

def _as_f64(X):
    return np.asarray(X, dtype=np.float64)


def matmul_numpy(A, B, n_slices=8, safe_mode="raise", pipeline="host",
                 precision="high"):
    """matmul.py:854-900 (and :731-778 for pipeline='ondevice')."""
    A = _as_f64(A)
    B = _as_f64(B)
    if pipeline == "ondevice":
        n_hi, n_lo = resolve_precision(precision)
        return matmul_ondevice_a3(A, B, safe_mode, n_hi, n_lo)
    if pipeline != "host":
        raise ValueError(
            f"Unknown pipeline={pipeline!r}; expected 'host' or 'ondevice'.")
    rep = host_safety_report(A, B, n_slices)
    fb = handle_unsafe(A, B, rep, safe_mode)
    if fb is not None:
        return fb
    a, ae, b, be = host_slices(A, B, rep["rho"], n_slices)
    sched = host_schedule(n_slices)
    return accumulate_a1(slice_products(a, b, sched), sched, ae, be)


def matmul_host_a2(A, B, n_slices=8, safe_mode="raise"):
    """matmul.py:826-851: what `matmul(pipeline='host')` returns (order A2)."""
    A = _as_f64(A)
    B = _as_f64(B)
    rep = host_safety_report(A, B, n_slices)
    fb = handle_unsafe(A, B, rep, safe_mode)
    if fb is not None:
        return fb
    a, ae, b, be = host_slices(A, B, rep["rho"], n_slices)
    sched = host_schedule(n_slices)
    return accumulate_a2(slice_products(a, b, sched), sched, ae, be)


def matmul_ondevice_a3(A, B, safe_mode="raise", n_hi=4, n_lo=1):
    """matmul.py:731-778: matmul_numpy(pipeline='ondevice') (order A3); also
    what matmul(pipeline='ondevice', accumulation='host') returns
    (matmul.py:688-728)."""
    A = _as_f64(A)
    B = _as_f64(B)
    rep = ondevice_safety_report(A, B, n_hi, n_lo)
    fb = handle_unsafe(A, B, rep, safe_mode)
    if fb is not None:
        return fb
    a, ae, b, be = ondevice_slices(A, B, rep["rho"], n_hi, n_lo)
    sched = ondevice_schedule(n_hi, n_lo)
    return accumulate_a3(slice_products(a, b, sched), sched, ae, be)


def matmul_ondevice_a4(A, B, safe_mode="raise", n_hi=4, n_lo=1,
                       return_pair=False):
    """matmul.py:641-686 with accumulation in {'fused', 'bf16_interleaved',
    'ondevice'}: split + FP32 extraction + products + A4 + FP64 combine
    (matmul.py:514-540, :711-722).  NumPy extraction semantics (extract.py:
    116-191) are used for the exponent (np.log2)."""
    A = _as_f64(A)
    B = _as_f64(B)
    rep = ondevice_safety_report(A, B, n_hi, n_lo)
    fb = handle_unsafe(A, B, rep, safe_mode)
    if fb is not None:
        return fb
    return _ozaki_a4_unchecked(A, B, rep["rho"], n_hi, n_lo, return_pair)


def _ozaki_a4_unchecked(A, B, rho, n_hi, n_lo, return_pair=False):
    a, ae, b, be = ondevice_slices(A, B, rho, n_hi, n_lo)
    sched = ondevice_schedule(n_hi, n_lo)
    ch, cl = accumulate_a4(slice_products(a, b, sched), sched, ae, be)
    if return_pair:
        return ch, cl
    return combine_f64(ch, cl)


def gram_ozaki(A, precision="high"):
    """gram.py:19-37, :92-95: G = Ozaki(A^T, A) (A4), rho from A.shape[0],
    then (G + G^T) * 0.5."""
    A = _as_f64(A)
    if A.ndim != 2:
        raise ValueError(f"A must be 2D, got ndim={A.ndim}.")
    n_hi, n_lo = resolve_precision(precision)
    rho = rho_f32(A.shape[0])
    G = _ozaki_a4_unchecked(np.ascontiguousarray(A.T), A, rho, n_hi, n_lo)
    return (G + G.T) * 0.5


def ozaki_matvec(A, x2, rho, n_hi, n_lo):
    """solve.py:38-53: A @ x with x as (K, cols), A4 order."""
    return _ozaki_a4_unchecked(A, x2, rho, n_hi, n_lo)


def residual_ozaki(A, x, b, precision="high"):
    """solve.py:78-82, :91-151 in mode='ozaki': b - Ozaki(A, x),
    rho from A.shape[1]."""
    A = _as_f64(A)
    x = _as_f64(x)
    b = _as_f64(b)
    n_hi, n_lo = resolve_precision(precision)
    vec = x.ndim == 1
    x2 = x[:, None] if vec else x
    b2 = b[:, None] if vec else b
    rho = rho_f32(A.shape[1])
    r = b2 - ozaki_matvec(A, x2, rho, n_hi, n_lo)
    return r[:, 0] if vec else r


def solve_ozaki(A, b, precision="high", max_iterations=3):
    """solve.py:154-167, :189-257 with residual_mode='ozaki': FP32 LU solve,
    then max_iterations x {r = b - Ozaki(A, x); x += f64(solve32(A, r))}."""
    A = _as_f64(A)
    b = _as_f64(b)
    n_hi, n_lo = resolve_precision(precision)
    vec = b.ndim == 1
    b2 = b[:, None] if vec else b
    rho = rho_f32(A.shape[0])
    A32 = A.astype(np.float32)
    x = np.linalg.solve(A32, b2.astype(np.float32)).astype(np.float64)
    for _ in range(max_iterations):
        r = b2 - ozaki_matvec(A, x, rho, n_hi, n_lo)
        x = x + np.linalg.solve(A32, r.astype(np.float32)).astype(np.float64)
    return x[:, 0] if vec else x
